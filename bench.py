"""Benchmark of the gfx950 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-secondary]

Headline workload: bf16 matmul C = A @ B, M = N = K = 4096,
row-major, fp32 accumulation, bf16 output, A and B ~ N(0,1)*0.02 (synthetic, resident in
HBM before timing). One step = one launch of the matmul entry through the C ABI on
torch's current stream; W untimed warm-up steps (default 500), continued until at least
HEADLINE_WARMUP_S = 0.2 s of them have run (MI355X raises its clock over the first tens of
milliseconds of sustained load: after 5 launches the same kernel times 1158 TFLOP/s, after
0.05-1.6 s of launches 1320-1355), then exactly K timed steps (default 200) bracketed by
torch.cuda.synchronize().
value = algorithmic FLOP (2*M*N*K) per step / step time.

The JSON line also carries
  roofline: the GEMM kernel against dense bf16 MFMA peak, from HIP events on the launch
            stream; traffic (HBM bytes per launch) from the rocprofv3 PMC summary in
            profiles/ when present;
  cpu_baseline: the oracle's restatement of the reference's npu_demo matmul loop nest,
            compiled without optimisation like the reference (g++ -shared -fPIC, no -O)
            and run on 2 host threads (npu_demo block_num = 2) over a bounded sample of
            the same workload (the first 384 output rows), plus the same sample built with
            -O2 (optimized_value) and the host CPU model;
  secondary: the other BASELINE configs (C1, C2', C3, C4, C5 D=128/64) and two fp32 extension
            lines (C2's and C4's shapes in the reference demos' fp32), each after 0.15 s
            of untimed launches, over >= 200 (C1, C2'), 1000 (C3), 100 (C4), 25 (C5), 50
            (fp32 matmul) or 20 (fp32 attention) back-to-back launches. Each carries its
            own cpu_baseline: the same restated loop nest (-O0, 2 threads), C1 in full
            (median of 5), the others on a fixed sample of outer tiles extrapolated to the
            full problem (cpu_baselines()).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT))

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16/fp16 MFMA (256 CU x 4096 FLOP/clk x 2.4 GHz)
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
METRIC = "TFLOP/s & % bf16 MFMA peak: 4096^3 matmul, flash-attn fwd S=2048 D=128"
GEMM_TRAFFIC_FILE = REPO_ROOT / "profiles" / "gemm_bf16_4096_traffic.txt"
HEADLINE_WARMUP_S = 0.2  # untimed launches before the headline's timed steps, at least this long


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class PreparedCall:
    """An entry point with its slot array marshalled once (launch cost = one ctypes call)."""

    def __init__(self, entry: str, args) -> None:
        from kernelcode_generate_amd import native

        self.lib = native.load_library()
        self.fn = getattr(self.lib, entry)
        self.slots, self._keep = native.marshal_slots(args)
        self.count = len(args)
        self.entry = entry

    def __call__(self) -> None:
        rc = self.fn(self.slots, self.count)
        if rc != 0:
            raise RuntimeError(f"{self.entry} returned {rc}: {self.lib.kg_gfx950_last_error().decode()}")


PROBE_LIBRARY = REPO_ROOT / "kernelcode_generate_amd" / "libkg_gfx950_probe.so"
_PROBE = None


def probe_library():
    """bench.py's measurement library (built next to libkg_gfx950.so by build()), loaded
    after the product library so that both use torch's HIP runtime."""

    global _PROBE
    if _PROBE is None:
        import ctypes

        from kernelcode_generate_amd import native

        native.load_library()
        if not PROBE_LIBRARY.is_file():
            raise RuntimeError(f"{PROBE_LIBRARY} is missing: build it with __graft_entry__.build()")
        lib = ctypes.CDLL(str(PROBE_LIBRARY))
        lib.kg_gfx950_probe_mfma_rate.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_double)] * 2
        lib.kg_gfx950_probe_mfma_rate.restype = ctypes.c_int
        lib.kg_gfx950_probe_last_error.restype = ctypes.c_char_p
        _PROBE = lib
    return _PROBE


def mfma_rate(dtype: str = "bf16", zero_operands: bool = False, iterations: int = 20000, workgroups: int = 2048,
              mfma_m: int = 16) -> dict:
    """Sustained rate of v_mfma_f32_16x16x32 (mfma_m=16) or v_mfma_f32_32x32x16 (mfma_m=32)
    on register operands, N(0,1)*0.02 or zeros (the probe library's kg_gfx950_probe_mfma_rate)."""

    import ctypes

    lib = probe_library()
    tf, ghz = ctypes.c_double(0.0), ctypes.c_double(0.0)
    code = {"bf16": 6, "f16": 5}[dtype]
    rc = lib.kg_gfx950_probe_mfma_rate(code, int(mfma_m), int(bool(zero_operands)), int(iterations), int(workgroups),
                                       ctypes.byref(tf), ctypes.byref(ghz))
    if rc != 0:
        raise RuntimeError(f"kg_gfx950_probe_mfma_rate failed ({rc}): {lib.kg_gfx950_probe_last_error().decode()}")
    return {"tflops": tf.value, "clock_ghz": ghz.value}


def time_steps(call: PreparedCall, steps: int, warmup: int, min_warmup_s: float = 0.0):
    """Return (wall ms per step, event ms per step, warmup launches) over exactly `steps`
    launches, after `warmup` untimed launches and, if min_warmup_s > 0, more untimed
    launches until that much time has passed. MI355X raises its clock over the first tens
    of milliseconds of sustained load (C4: 299 us per launch over the first 20 launches,
    251 us after 150), so a short warm-up times the clock ramp, not the kernel."""

    import torch

    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    if min_warmup_s > 0:
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < min_warmup_s:
            for _ in range(16):
                call()
            torch.cuda.synchronize()
            warmup += 16
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        call()
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_time(e1) / steps, warmup


def read_traffic(path: Path):
    if not path.is_file():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text())
    return float(m.group(1)) if m else None


def gemm_workload(dev, m: int, n: int, k: int, seed: int):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    a = (torch.randn(m, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b = (torch.randn(k, n, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    c = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    return a, b, c


def cpu_baseline_matmul(rows: int = 384):
    import numpy as np

    import oracle

    rng = np.random.default_rng(20261202)
    a = (rng.standard_normal((4096, 4096), dtype=np.float32) * 0.02)
    b = (rng.standard_normal((4096, 4096), dtype=np.float32) * 0.02)
    oracle.matmul_demo(a[:48], b, None, (48, 80, 56), threads=2, m_range=(0, 48), optimized=False)  # warm
    t0 = time.perf_counter()
    oracle.matmul_demo(a, b, None, (48, 80, 56), threads=2, m_range=(0, rows), optimized=False)
    dt = time.perf_counter() - t0
    flop = 2.0 * rows * 4096 * 4096
    # the same sample through the same loop nest built with optimisation
    t0 = time.perf_counter()
    oracle.matmul_demo(a, b, None, (48, 80, 56), threads=2, m_range=(0, rows), optimized=True)
    dt_opt = time.perf_counter() - t0
    return {
        "value": flop / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 2,
        "kind": "port",
        "sample": f"output rows 0-{rows - 1} of the 4096^3 matmul ({flop / 1e9:.1f} GFLOP) through the restated "
                  f"npu_demo tile loop (tiles 48x80x56, fp32, -O0 like the reference's build, 2 threads): {dt:.2f} s",
        "optimized_value": flop / dt_opt / 1e12,
        "optimized_sample": f"the same rows built with -O2: {dt_opt:.2f} s",
        "host_cpus": os.cpu_count(),
        "cpu_model": cpu_model(),
    }


def _timed(fn, repeats: int = 1) -> float:
    """Median wall seconds of `repeats` calls of fn."""

    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def cpu_baselines(keys) -> dict:
    """CPU baseline of every secondary workload: the oracle's restatement of the
    reference's npu_demo loop nest for it (kernel/{matmul,conv2d,flash_attention}/
    inputs_static_tile_static.py on include/npu_demo/Kernel.h), compiled without -O like
    the reference's build and run on 2 host threads (npu_demo block_num = 2, the
    block-strided top-level loop). C1 runs in full (median of 5); the others run a fixed
    sample of outer tiles and are extrapolated to the full problem by algorithmic FLOP
    (causal: kept query-key pairs), labelled "extrapolated". Inputs have the workloads'
    shapes and distributions (numpy generators, same seeds)."""

    import numpy as np

    import oracle

    out = {}
    model = cpu_model()

    def rec(value_flop, seconds, full_flop, sample, cores=2, extrapolated=True):
        r = {"value": value_flop / seconds / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
             "sample": sample, "sample_s": round(seconds, 3), "extrapolated": extrapolated,
             "full_problem_s": round(full_flop / (value_flop / seconds), 2), "cpu_model": model}
        return r

    tiles_mm = (48, 80, 56)
    if "c1" in keys:
        rng = np.random.default_rng(20261201)
        a = rng.uniform(-1, 1, (256, 256)).astype(np.float32)
        b = rng.uniform(-1, 1, (256, 256)).astype(np.float32)
        oracle.matmul_demo(a, b, None, tiles_mm, threads=2, optimized=False)  # warm
        dt = _timed(lambda: oracle.matmul_demo(a, b, None, tiles_mm, threads=2, optimized=False), 5)
        f = 2.0 * 256**3
        out["c1"] = rec(f, dt, f, "the whole 256^3 fp32 matmul through the restated npu_demo tile loop "
                        "(tiles 48x80x56), median of 5 runs", extrapolated=False)
    if "c2s" in keys:
        rng = np.random.default_rng(20261203)
        rows = 128
        a = rng.standard_normal((rows, 4096), dtype=np.float32) * 0.02
        b = rng.standard_normal((4096, 1024), dtype=np.float32) * 0.02
        dt = _timed(lambda: oracle.matmul_demo(a, b, None, tiles_mm, threads=2, optimized=False))
        out["c2s"] = rec(2.0 * rows * 1024 * 4096, dt, 2.0 * 8192 * 1024 * 4096,
                         f"output rows 0-{rows - 1} of 8192 (tiles 48x80x56, fp32)")
    if "c3" in keys:
        rng = np.random.default_rng(20261204)
        x = rng.standard_normal((32, 64, 56, 56), dtype=np.float32)
        bound = math.sqrt(6.0 / 576.0)
        w = rng.uniform(-bound, bound, (64, 64, 3, 3)).astype(np.float32)
        nf = 16
        dt = _timed(lambda: oracle.conv2d_demo(x, w, None, (1, 1), (1, 1), (1, 1, 1, 1), (8, 16, 4, 8, 9), threads=2,
                                               f_range=(0, nf), optimized=False))
        full = 2.0 * 32 * 64 * 56 * 56 * 64 * 9
        out["c3"] = rec(full * nf / 64, dt, full, f"filters 0-{nf - 1} of 64 (2 of 8 outer filter tiles; "
                        "tiles f8 c16 n4 ho8 wo9, fp32 img2col + matmul)")
    if "c4" in keys:
        rng = np.random.default_rng(20261205)
        heads, rows = 8, 128
        q, k, v = (rng.standard_normal((4, heads, 2048, 128), dtype=np.float32) for _ in range(3))
        dt = _timed(lambda: oracle.flash_attention_demo(q, k, v, 64, 80, scale=1 / math.sqrt(128), threads=2,
                                                        m_range=(0, rows), optimized=False))
        full = 4.0 * 4 * 32 * 2048 * 2048 * 128
        out["c4"] = rec(full * (heads / 32) * (rows / 2048), dt, full,
                        f"query rows 0-{rows - 1} of {heads} of 32 heads, all 4 batches (tiles br64 bc80, fp32)")
    for d, key, seed in ((128, "c5d128", 20261206), (64, "c5d64", 20261207)):
        if key not in keys:
            continue
        rng = np.random.default_rng(seed)
        heads, r0, r1 = 4, 8192, 8320
        q, k, v = (rng.standard_normal((1, heads, 16384, d), dtype=np.float32) for _ in range(3))
        dt = _timed(lambda: oracle.flash_attention_demo(q, k, v, 64, 80, scale=1 / math.sqrt(d), causal=True,
                                                        threads=2, m_range=(r0, r1), optimized=False))
        kept = sum(i + 1 for i in range(r0, r1))  # query-key pairs the mask keeps in the sample, per head
        full = 4.0 * 32 * 16384 * 16384 * d / 2
        # B = 1: the block-strided loop over batches gives one of the two threads work
        out[key] = rec(4.0 * d * heads * kept, dt, full,
                       f"query rows {r0}-{r1 - 1} of {heads} of 32 heads (causal: extrapolated by kept "
                       f"query-key pairs; tiles br64 bc80, fp32; B=1 leaves one of the 2 threads idle)", cores=1)
    return out


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


SECONDARY_KEYS = ("c1", "c2s", "c3", "c4", "c5d128", "c5d64", "f32gemm", "f32fa", "perop")
PROFILE_KEYS = ("c2",) + SECONDARY_KEYS  # --only also takes the headline GEMM, for counter runs


SECONDARY_WARMUP_S = 0.15  # untimed back-to-back launches per secondary workload, seconds


def secondary(dev, steps: int, warmup: int, only=None):
    import torch

    out = []
    keys = set(SECONDARY_KEYS if only is None else only)
    current = [None]

    def add(name, flop, call, peak, nsteps, byts=None, traffic_file=None):
        wall, ev, nwarm = time_steps(call, nsteps, min(warmup, 10), SECONDARY_WARMUP_S)
        tf = flop / (ev * 1e-3) / 1e12
        rec = {"key": current[0], "workload": name, "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ev, 5),
               "frac_of_peak": round(tf / peak, 4), "peak": peak, "steps": nsteps, "warmup_launches": nwarm}
        if byts is not None:
            gbs = byts / (ev * 1e-3) / 1e9
            rec["hbm_gbs"] = round(gbs, 1)
            rec["hbm_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        if traffic_file is not None:
            rec["traffic"] = read_traffic(REPO_ROOT / "profiles" / traffic_file)  # measured HBM bytes per launch
        log(f"[bench] {name}: {ev * 1e3:.1f} us  {tf:.1f} TFLOP/s  wall/step {wall * 1e3:.1f} us")
        out.append(rec)

    runs = {"c1": lambda: c1(dev, add, steps), "c2": lambda: c2(dev, add, steps), "c2s": lambda: c2s(dev, add, steps), "c3": lambda: c3(dev, add, steps),
            "c4": lambda: c4(dev, add, steps), "c5d128": lambda: c5(dev, add, steps, 128),
            "c5d64": lambda: c5(dev, add, steps, 64), "f32gemm": lambda: f32_gemm(dev, add, steps),
            "f32fa": lambda: f32_fa(dev, add, steps), "perop": lambda: perop_matmul(dev, add, steps)}
    for key in PROFILE_KEYS:
        if key in keys:
            current[0] = key
            runs[key]()
    return out


def c1(dev, add, steps):
    import torch

    g = torch.Generator(device=dev).manual_seed(20261201)
    a = torch.rand(256, 256, generator=g, device=dev) * 2 - 1
    b = torch.rand(256, 256, generator=g, device=dev) * 2 - 1
    c = torch.empty(256, 256, device=dev)
    add("C1 fp32 matmul 256^3", 2 * 256**3, PreparedCall("kg_gfx950_matmul_entry", (c, a, b, None)), PEAK_FP32_TFLOPS,
        max(steps, 200))


def c2(dev, add, steps):
    a, b, c = gemm_workload(dev, 4096, 4096, 4096, 20261202)
    add("C2 bf16 matmul M=N=K=4096", 2 * 4096**3, PreparedCall("kg_gfx950_matmul_entry", (c, a, b, None)),
        PEAK_BF16_TFLOPS, max(steps, 200))


def c2s(dev, add, steps):
    a, b, c = gemm_workload(dev, 8192, 1024, 4096, 20261203)
    add("C2' bf16 matmul M=8192 N=1024 K=4096", 2 * 8192 * 1024 * 4096,
        PreparedCall("kg_gfx950_matmul_entry", (c, a, b, None)), PEAK_BF16_TFLOPS, max(steps, 200))


def c3(dev, add, steps):
    import torch

    g = torch.Generator(device=dev).manual_seed(20261204)
    x = torch.randn(32, 64, 56, 56, generator=g, device=dev).to(torch.float16)
    bound = math.sqrt(6.0 / 576.0)
    w = ((torch.rand(64, 64, 3, 3, generator=g, device=dev) * 2 - 1) * bound).to(torch.float16)
    y = torch.empty(32, 64, 56, 56, dtype=torch.float16, device=dev)
    conv_bytes = 2 * (32 * 64 * 56 * 56 * 2) + 64 * 64 * 9 * 2
    add("C3 fp16 conv2d N=32 C=64 H=W=56 F=64 3x3 s1 p1", 2 * 32 * 64 * 56 * 56 * 64 * 9,
        PreparedCall("kg_gfx950_conv2d_entry", (y, x, w, None, 1, 1, 1, 1, 1, 1, 1, 1)), PEAK_BF16_TFLOPS,
        max(steps, 1000), conv_bytes, "conv2d_fp16_c3_traffic.txt")


def c4(dev, add, steps):
    import torch

    g = torch.Generator(device=dev).manual_seed(20261205)
    q, k, v = (torch.randn(4, 32, 2048, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    add("C4 bf16 flash-attn fwd B=4 H=32 S=2048 D=128 non-causal", 4 * 4 * 32 * 2048 * 2048 * 128,
        PreparedCall("kg_gfx950_flash_attention_entry", (o, q, k, v, 128, 64, 1.0 / math.sqrt(128.0), 0)),
        PEAK_BF16_TFLOPS, max(steps, 100), None, "flash_attn_bf16_c4_traffic.txt")


def c5(dev, add, steps, d):
    import torch

    seed = 20261206 if d == 128 else 20261207
    g = torch.Generator(device=dev).manual_seed(seed)
    q, k, v = (torch.randn(1, 32, 16384, d, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    o = torch.empty_like(q)
    add(f"C5 bf16 flash-attn fwd B=1 H=32 S=16384 D={d} causal", 4 * 32 * 16384 * 16384 * d // 2,
        PreparedCall("kg_gfx950_flash_attention_entry", (o, q, k, v, 128, 64, 1.0 / math.sqrt(d), 1)),
        PEAK_BF16_TFLOPS, max(20, steps // 4))


def perop_matmul(dev, add, steps):
    """The per-operation path, what a kernel the fuse pass does not recognise runs on: this
    package's tiled matmul program lowered with fuse=false (one HIP kernel executing the IR's
    operations on tiles, the reference's sequential-k fp32 arithmetic), compiled by the
    execution engine and called through its kg_execute_entry (workspace allocation included),
    fp32 1024^3 with 64 x 64 x 64 tiles; the fused library kernel on the same call follows."""

    import ctypes

    import torch

    from kernelcode_generate_amd import native
    from kernelcode_generate_amd.dsl import mlir_gen
    from kernelcode_generate_amd.execute_engine import ExecutionEngine
    from kernelcode_generate_amd.gen_kernel import gen_kernel
    from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_dynamic import (
        matmul_inputs_static_tile_dynamic_kernel as program,
    )
    from kernelcode_generate_amd.pipeline import get_pipeline

    m = n = k = 1024
    g = torch.Generator(device=dev).manual_seed(20261206)
    a = torch.rand(m, k, generator=g, device=dev) * 2 - 1
    b = torch.rand(k, n, generator=g, device=dev) * 2 - 1
    c = torch.empty(m, n, device=dev)
    args = (c, a, b, None, 64, 64, 64)
    lowered = get_pipeline("gfx950-lowering", {"fuse": "false"}).run(mlir_gen(program, args))
    compiled = ExecutionEngine("gfx950").compile(source=gen_kernel(lowered), function=program.__name__)
    try:
        lib = ctypes.CDLL(compiled.soname_path)
        entry = lib.kg_execute_entry
        entry.argtypes = [ctypes.POINTER(native.KgArgSlot), ctypes.c_ulonglong]
        entry.restype = ctypes.c_int
        slots, keep = native.marshal_slots(args)

        def call():
            if entry(slots, len(args)) != 0:
                raise RuntimeError(f"per-operation kg_execute_entry failed: {native.last_error()}")

        add("per-operation path: fp32 matmul 1024^3, tiles 64 (unfused DSL program)", 2.0 * m * n * k, call,
            PEAK_FP32_TFLOPS, max(10, steps // 10))
        add("fused library kernel on the same call (fp32 matmul 1024^3)", 2.0 * m * n * k,
            PreparedCall("kg_gfx950_matmul_entry", args), PEAK_FP32_TFLOPS, max(20, steps // 4))
        del keep
    finally:
        compiled.close()


def f32_gemm(dev, add, steps):
    """Extension: C2's shape with fp32 operands (the reference demos' dtype) on matrix cores."""
    import torch

    g = torch.Generator(device=dev).manual_seed(20261208)
    a, b = (torch.rand(4096, 4096, generator=g, device=dev) * 2 - 1 for _ in range(2))
    c = torch.empty(4096, 4096, device=dev)
    add("fp32 matmul M=N=K=4096 (extension: C2 shape in the demos' fp32)", 2 * 4096**3,
        PreparedCall("kg_gfx950_matmul_entry", (c, a, b, None)), PEAK_FP32_TFLOPS, max(20, steps // 4))


def f32_fa(dev, add, steps):
    """Extension: C4's shape with fp32 Q/K/V on matrix cores."""
    import torch

    g = torch.Generator(device=dev).manual_seed(20261209)
    q, k, v = (torch.randn(4, 32, 2048, 128, generator=g, device=dev) for _ in range(3))
    o = torch.empty_like(q)
    add("fp32 flash-attn fwd B=4 H=32 S=2048 D=128 non-causal (extension: C4 shape in fp32)",
        4 * 4 * 32 * 2048 * 2048 * 128,
        PreparedCall("kg_gfx950_flash_attention_entry", (o, q, k, v, 64, 64, 1.0 / math.sqrt(128.0), 0)),
        PEAK_FP32_TFLOPS, max(10, steps // 10))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed launches of the headline GEMM")
    ap.add_argument("--warmup", type=int, default=500,
                    help="untimed launches before them (500 x ~115 us: the clock has settled)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", nargs="+", choices=PROFILE_KEYS,
                    help="profiling aid: run only these secondary workloads (no headline GEMM, no CPU baseline)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one MI355X: the gfx950 hot-path kernels are single-GPU and this build has no "
            "multi-GPU path. Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from kernelcode_generate_amd import native

    dev = torch.device("cuda:0")
    native.load_library()
    stream = torch.cuda.current_stream()
    native.set_launch_mode(False, stream.cuda_stream)
    if args.only:
        print(json.dumps({"secondary": secondary(dev, args.steps, args.warmup, args.only)}), flush=True)
        native.set_launch_mode(True, None)
        return 0

    m = n = k = 4096
    a, b, c = gemm_workload(dev, m, n, k, 20261202)
    call = PreparedCall("kg_gfx950_matmul_entry", (c, a, b, None))
    torch.cuda.synchronize()
    wall_ms, ev_ms, warm_launches = time_steps(call, args.steps, args.warmup, HEADLINE_WARMUP_S)
    flop = 2.0 * m * n * k
    value = flop / (wall_ms * 1e-3) / 1e12
    achieved = flop / (ev_ms * 1e-3) / 1e12
    log(f"[bench] C2 bf16 matmul 4096^3: kernel {ev_ms * 1e3:.1f} us ({achieved:.1f} TFLOP/s), wall/step {wall_ms * 1e3:.1f} us")
    traffic = read_traffic(GEMM_TRAFFIC_FILE)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_launches": warm_launches,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: A,B ~ N(0,1)*0.02 (seeded torch generator on the device), resident in HBM",
        "config": {
            "workload": "bf16 matmul M=N=K=4096, row-major A[M,K] B[K,N], fp32 accumulate, bf16 out (BASELINE configs[1])",
            "M": m, "N": n, "K": k,
            "kernel": "gemm_quad_kernel: 256x256 tiles, 4 waves of 128x128 (fp32 accumulators in AGPRs), "
                      "4-stage HBM->LDS ring, v_mfma_f32_16x16x32_bf16, C stored through LDS as whole row segments",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "algorithmic_flop_per_launch": flop,
            "avg_launch_ms": round(ev_ms, 5),
        },
    }
    del a, b, c
    # the part's sustained matrix-core rate on this data (random bf16, no operand movement):
    # the power-limited ceiling the headline's fraction is read against
    ceiling = mfma_rate("bf16", False, mfma_m=16)
    result["roofline"]["mfma_ceiling"] = {
        "tflops": round(ceiling["tflops"], 1), "clock_ghz": round(ceiling["clock_ghz"], 3),
        "what": "back-to-back v_mfma_f32_16x16x32_bf16 (the headline kernel's instruction) on N(0,1)*0.02 "
                "register operands (the probe library's kg_gfx950_probe_mfma_rate)"}
    result["roofline"]["frac_of_mfma_ceiling"] = round(achieved / ceiling["tflops"], 4)
    log(f"[bench] mfma ceiling (random bf16 operands): {ceiling['tflops']:.1f} TFLOP/s at {ceiling['clock_ghz']:.3f} GHz; "
        f"headline {achieved / ceiling['tflops']:.3f} of it")
    if not args.no_secondary:
        result["secondary"] = secondary(dev, max(5, args.steps // 2), args.warmup)
    native.set_launch_mode(True, None)
    if not args.no_cpu_baseline:
        cb = cpu_baseline_matmul()
        log(f"[bench] cpu baseline: {cb['value'] * 1e3:.3f} GFLOP/s ({cb['sample']})")
        result["cpu_baseline"] = cb
        if "secondary" in result:
            # the fp32 extension lines share C2's and C4's loop nests: their baselines are those
            keys = {r["key"] for r in result["secondary"]}
            baselines = cpu_baselines(keys | ({"c4"} if "f32fa" in keys else set()))
            baselines["f32gemm"] = dict(cb, note="the headline's sample: the same 4096^3 loop nest in fp32")
            baselines["perop"] = dict(cb, note="the headline's sample: the same matmul loop nest in fp32")
            if "c4" in baselines:
                baselines["f32fa"] = dict(baselines["c4"], note="C4's sample: the same loop nest in fp32")
            for r in result["secondary"]:
                if r["key"] in baselines:
                    r["cpu_baseline"] = baselines[r["key"]]
                    b = baselines[r["key"]]
                    how = f"{b['sample_s']} s" if "sample_s" in b else b.get("note", "")
                    log(f"[bench] cpu baseline {r['key']}: {b['value'] * 1e3:.3f} GFLOP/s ({how})")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
