"""The cost model against the GPU (the gfx950 analogue of dsl_cost_run,
kernel_gen/tools/dsl_run.py:656-730): every case of tests/cost_cases.py (each kernel choice
of the library) is run and timed with HIP events, and

  - the modelled MFMA cycles carry at least the operation's FLOP (2 per MAC; a SIMD does
    1024 16-bit MFMA FLOP per cycle in either shape, 32x32x16 or 16x16x32, and 64 fp32 FLOP
    per cycle of 32x32x2), exactly on exact-tile shapes;
  - no case runs faster than its ROOFLINE_NS (matrix-core time of the modelled MFMAs at the
    2.4 GHz peak clock, or compulsory HBM bytes at 8 TB/s), less 10 % for timer resolution;
  - cases whose roofline is at least 20 us run within 4x of it (the stated band: these
    kernels reach 25 % or more of the roofline; the counted instruction totals themselves
    are pinned by profiles/mfma_instruction_counts.txt).
"""

from __future__ import annotations

import pytest

from kernelcode_generate_amd import native
from kernelcode_generate_amd.tools import roofline_ns
from tests.cost_cases import CASES, modelled, prepare

pytestmark = pytest.mark.gpu
FLOP_PER_MFMA_CYCLE = {"float32": 64, "bfloat16": 1024, "float16": 1024}
EXACT = {"gemm_bf16_4096", "gemm_bf16_c2s_8192x1024x4096", "gemm_f16_512x768x256", "gemm_f32_256",
         "gemm_f32_splitk_512x512x4096", "gemm_f32_mfma_1024x256x1024"}


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_cost_model_against_the_gpu(device, case):
    import torch

    name, family, dtype = case[0], case[1], case[2]
    model = modelled(case)
    if model["MFMA"]:
        assert model["MFMA_CYCLES"] * FLOP_PER_MFMA_CYCLE[dtype] >= 2 * model["MAC"], name
        if name in EXACT:
            assert model["MFMA_CYCLES"] * FLOP_PER_MFMA_CYCLE[dtype] == 2 * model["MAC"], name
    roof = roofline_ns(model)
    print(f"[cost] {name}: roofline {roof} ns", flush=True)
    entry, args = prepare(case)
    native.call_entry(entry, args)  # warm
    # back-to-back launches enqueued on one stream: the host's validation of call i+1
    # overlaps the kernel of call i, so the events see kernel time
    stream = torch.cuda.current_stream()
    native.set_launch_mode(False, stream.cuda_stream)
    try:
        launches = 20
        for _ in range(launches):
            native.call_entry(entry, args)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(launches):
            native.call_entry(entry, args)
        e1.record(stream)
        e1.synchronize()
    finally:
        native.set_launch_mode(True, None)
    measured = e0.elapsed_time(e1) * 1e6 / launches
    print(f"[cost] {name}: measured {measured:.0f} ns ({roof / measured:.2f} of the roofline)", flush=True)
    assert measured >= 0.9 * roof, f"{name}: {measured:.0f} ns beats the modelled roofline {roof} ns"
    if roof >= 20_000:
        assert measured <= 4 * roof, f"{name}: {measured:.0f} ns is more than 4x the roofline {roof} ns"
    assert native.last_error() == ""


@pytest.mark.gpu
def test_mfma_rate_measures_the_matrix_cores(device):
    """bench.py's MFMA-rate probe (its own library, not the product's): a short run gives a
    rate below the nominal dense peak and above a tenth of it, for both MFMA shapes and both
    operand kinds, and a clock within the part's range."""
    import bench

    for mfma_m in (16, 32):
        for zeros in (False, True):
            r = bench.mfma_rate("bf16", zeros, iterations=2000, workgroups=1024, mfma_m=mfma_m)
            print(f"[mfma_rate] m={mfma_m} zeros={zeros}: {r['tflops']:.0f} TFLOP/s at {r['clock_ghz']:.2f} GHz",
                  flush=True)
            assert 0.1 * 2516.6 < r["tflops"] < 2516.6
            assert 0.5 < r["clock_ghz"] < 2.6
