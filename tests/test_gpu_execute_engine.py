"""GPU tests of the drop-in path: every demo kernel through run_gfx950_demo / dsl_run ->
gfx950-lowering -> generated SourceBundle -> hipcc -> ctypes kg_execute_entry, with the
inputs of the reference's runtime test (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:
499-597: numpy arange matmul/conv inputs, default_rng(2026052901) attention inputs) and
expected values from the closed forms that test uses."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd.core.config import restore_config, set_target, snapshot_config
from kernelcode_generate_amd.execute_engine import ExecuteRequest
from kernelcode_generate_amd.kernel.conv2d.inputs_dynamic_tile_dynamic import conv2d_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_dynamic import conv2d_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_static import conv2d_inputs_static_tile_static_kernel
from kernelcode_generate_amd.kernel.flash_attention.inputs_dynamic_tile_dynamic import (
    flash_attention_inputs_dynamic_tile_dynamic_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.inputs_static_tile_dynamic import (
    flash_attention_inputs_static_tile_dynamic_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.inputs_static_tile_static import (
    flash_attention_inputs_static_tile_static_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.scaled import (
    flash_attention_scaled_causal_kernel,
    flash_attention_scaled_kernel,
)
from kernelcode_generate_amd.kernel.matmul.inputs_dynamic_tile_dynamic import matmul_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_dynamic import matmul_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_static import matmul_inputs_static_tile_static_kernel
from kernelcode_generate_amd.kernel.runner import run_gfx950_demo
from kernelcode_generate_amd.tools import dsl_run
from tests.golden.make_golden import attention_closed_form, conv_closed_form
from tests.gpu_util import assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True)
def _config():
    snap = snapshot_config()
    yield
    restore_config(snap)


@pytest.mark.parametrize(
    "kernel,extra",
    [
        (matmul_inputs_static_tile_static_kernel, ()),
        (matmul_inputs_static_tile_dynamic_kernel, (2, 2, 2)),
        (matmul_inputs_dynamic_tile_dynamic_kernel, (2, 2, 2)),
    ],
    ids=lambda v: getattr(v, "__name__", str(v)),
)
def test_matmul_demos(device, kernel, extra):
    lhs = np.arange(6, dtype=np.float32).reshape(2, 3)
    rhs = np.arange(12, dtype=np.float32).reshape(3, 4)
    bias = np.arange(4, dtype=np.float32)
    print(f"[dsl_run] {kernel.__name__}", flush=True)
    absent = np.zeros((2, 4), np.float32)
    present = np.zeros((2, 4), np.float32)
    r1 = run_gfx950_demo("matmul/absent", kernel, (absent, lhs, rhs, None, *extra), absent, lhs @ rhs, atol=1e-5, rtol=1e-5)
    r2 = run_gfx950_demo("matmul/present", kernel, (present, lhs, rhs, bias, *extra), present, lhs @ rhs + bias,
                         atol=1e-5, rtol=1e-5)
    assert r1.dsl_result.execute_result.ok and r2.dsl_result.execute_result.ok
    assert r1.dsl_result.execute_result.elapsed_ms > 0.0


def _conv_case(xs, ws, stride, dil, pad):
    x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs)
    w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
    b = np.arange(ws[0], dtype=np.float32)
    return x, w, b, conv_closed_form(x, w, None, stride, dil, pad), conv_closed_form(x, w, b, stride, dil, pad)


def test_conv2d_static_static_demo(device):
    # module constants of the static demo: stride 8, pads (3,3,4,0), tiles (7,18,3,9,8);
    # the reference's case uses input (4,49,248,232) and weight (20,49,3,5)
    xs, ws, pad = (4, 49, 248, 232), (20, 49, 3, 5), (3, 3, 4, 0)
    x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs) / np.float32(1e6)
    w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
    b = np.arange(ws[0], dtype=np.float32)
    for bias in (None, b):
        exp = conv_closed_form(x, w, bias, (8, 8), (1, 1), pad)
        out = np.zeros(exp.shape, np.float32)
        run_gfx950_demo("conv/static", conv2d_inputs_static_tile_static_kernel, (out, x, w, bias), out, exp,
                        atol=1e-3, rtol=1e-4)


def test_conv2d_static_tile_dynamic_demo(device):
    from kernelcode_generate_amd.kernel.conv2d import inputs_static_tile_dynamic as mod

    pad = (mod._STATIC_PAD_TOP, mod._STATIC_PAD_BOTTOM, mod._STATIC_PAD_LEFT, mod._STATIC_PAD_RIGHT)
    x, w, b, exp_a, exp_p = _conv_case((1, 2, 21, 29), (3, 2, 2, 2), (8, 8), (1, 1), pad)
    for bias, exp in ((None, exp_a), (b, exp_p)):
        out = np.zeros(exp.shape, np.float32)
        run_gfx950_demo("conv/static_dyn", conv2d_inputs_static_tile_dynamic_kernel, (out, x, w, bias, 7, 18, 3, 9, 8), out,
                        exp, atol=1e-5, rtol=1e-5)


def test_conv2d_dynamic_demo(device):
    x, w, b, exp_a, exp_p = _conv_case((1, 2, 4, 5), (3, 2, 2, 2), (1, 1), (1, 1), (1, 1, 1, 1))
    for bias, exp in ((None, exp_a), (b, exp_p)):
        out = np.zeros(exp.shape, np.float32)
        run_gfx950_demo("conv/dyn", conv2d_inputs_dynamic_tile_dynamic_kernel,
                        (out, x, w, bias, 1, 1, 1, 1, 1, 1, 1, 1, 7, 18, 3, 9, 8), out, exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize(
    "kernel,extra",
    [
        (flash_attention_inputs_static_tile_static_kernel, ()),
        (flash_attention_inputs_static_tile_dynamic_kernel, (2, 2)),
        (flash_attention_inputs_dynamic_tile_dynamic_kernel, (2, 2)),
    ],
    ids=lambda v: getattr(v, "__name__", str(v)),
)
def test_flash_attention_demos(device, kernel, extra):
    v = dict(np.load(GOLDEN / "cuda_runtime_vectors.npz"))
    out = np.zeros_like(v["fa_q"])
    run_gfx950_demo("fa", kernel, (out, v["fa_q"], v["fa_k"], v["fa_v"], *extra), out, v["fa_expected"], atol=1e-4,
                    rtol=1e-4)


@pytest.mark.parametrize("kernel,causal", [(flash_attention_scaled_kernel, False),
                                           (flash_attention_scaled_causal_kernel, True)])
def test_scaled_attention_device_tensors(device, kernel, causal):
    """bf16 device tensors are used in place (no staging); D=128 takes the MFMA kernel."""

    import torch

    rng = np.random.default_rng(7)
    shape = (1, 2, 256, 128)
    (qt, q), (kt, k), (vt, vv) = (round_to(rng.standard_normal(shape, dtype=np.float32), torch.bfloat16) for _ in range(3))
    qd, kd, vd = qt.cuda(), kt.cuda(), vt.cuda()
    out = torch.empty_like(qd)
    scale = 1.0 / np.sqrt(128.0)
    snap = snapshot_config()
    set_target("gfx950")
    try:
        result = dsl_run(kernel, (out, qd, kd, vd, 128, 64, scale), "gfx950-lowering")
    finally:
        restore_config(snap)
    assert result.execute_result.ok and result.execute_result.elapsed_ms > 0
    assert_h16_close(to_numpy(out), attention_closed_form(q, k, vv, scale, causal), what=kernel.__name__)


def test_stream_execution(device):
    import torch

    set_target("gfx950")
    a = torch.randn(512, 256, device="cuda").to(torch.bfloat16)
    b = torch.randn(256, 512, device="cuda").to(torch.bfloat16)
    out = torch.empty(512, 512, device="cuda", dtype=torch.bfloat16)
    result = dsl_run(matmul_inputs_static_tile_dynamic_kernel, (out, a, b, None, 64, 64, 64), "gfx950-lowering")
    kernel = result.compiled_kernel
    out2 = torch.zeros_like(out)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        r = kernel.execute(request=ExecuteRequest(args=(out2, a, b, None, 64, 64, 64), stream=stream))
    stream.synchronize()
    assert r.ok
    assert torch.equal(out, out2)


def test_memory_stage_pipeline_option(device):
    """gfx950-lowering{memory_stage=2}: the generated entry forwards the ring depth to the
    library, and the result is the default pipeline's, bit for bit."""

    import torch

    from kernelcode_generate_amd.pipeline import get_pipeline

    set_target("gfx950")
    a = torch.randn(512, 256, device="cuda").to(torch.bfloat16)
    b = torch.randn(256, 512, device="cuda").to(torch.bfloat16)
    out = torch.empty(512, 512, device="cuda", dtype=torch.bfloat16)
    out2 = torch.zeros_like(out)
    dsl_run(matmul_inputs_static_tile_dynamic_kernel, (out, a, b, None, 64, 64, 64), "gfx950-lowering")
    staged = dsl_run(matmul_inputs_static_tile_dynamic_kernel, (out2, a, b, None, 64, 64, 64),
                     get_pipeline("gfx950-lowering", {"memory_stage": "2"}))
    assert "slots[7].int_value = 2LL;" in staged.source
    assert torch.equal(out, out2)


# ------------------------------------------------------------------------------------
# the IR paths: fused and per-operation execution of the same DSL kernels
# ------------------------------------------------------------------------------------

from kernelcode_generate_amd.operation import kernel as dsl_kernel  # noqa: E402
from kernelcode_generate_amd.operation.dma import alloc, broadcast, deslice, view  # noqa: E402
from kernelcode_generate_amd.operation.scf import loop  # noqa: E402
from kernelcode_generate_amd.pipeline import get_pipeline  # noqa: E402
from kernelcode_generate_amd.symbol_variable import MemorySpace, NumericType, SymbolDim  # noqa: E402
from tests.test_dsl_frontend import my_gemm  # noqa: E402

PER_OP = {"fuse": "false"}


def _run(fn, args, options=None):
    set_target("gfx950")
    pipeline = get_pipeline("gfx950-lowering", options) if options else "gfx950-lowering"
    print(f"[dsl_run] {fn.__name__} {options or ''}", flush=True)
    return dsl_run(fn, tuple(args), pipeline)


@pytest.mark.parametrize("variant", ["static", "dyn", "dyn_chunks", "dyn_wide"])
def test_per_op_matmul_matches_oracle_bit_for_bit(device, oracle_mod, variant):
    """The per-operation path computes the demo's own loop nest (sequential-k fp32 products
    and sums, like include/npu_demo/Kernel.h:900-948): it reproduces the oracle exactly.
    The runtime's matmul stages its operands through LDS in k chunks of 4096 // max(M, N):
    one chunk for 50 x 64 x 17 tiles, three (32, 32, 16) for 96 x 128 x 80 tiles; tiles
    wider than 4096 read the operands in place. The workspace (the tiles) of the first two
    cases fits the 96 KiB the entry keeps in LDS; that of the last two is device memory."""

    from kernelcode_generate_amd.kernel.matmul import inputs_static_tile_static as mod

    m, k, n = (3, 40, 4500) if variant == "dyn_wide" else (97, 130, 75)
    rng = np.random.default_rng(21)
    lhs = rng.standard_normal((m, k), dtype=np.float32)
    rhs = rng.standard_normal((k, n), dtype=np.float32)
    bias = rng.standard_normal(n, dtype=np.float32)
    out = np.zeros((m, n), np.float32)
    if variant == "static":
        r = _run(matmul_inputs_static_tile_static_kernel, (out, lhs, rhs, bias), PER_OP)
        tiles = (mod._TILE_M, mod._TILE_N, mod._TILE_K)
    else:
        tiles = {"dyn": (50, 64, 17), "dyn_chunks": (96, 128, 80), "dyn_wide": (3, 4500, 40)}[variant]
        r = _run(matmul_inputs_dynamic_tile_dynamic_kernel, (out, lhs, rhs, bias, *tiles), PER_OP)
    assert r.fused is None and "kg_gfx950_generated_kernel" in r.source
    assert np.array_equal(out, oracle_mod.matmul_demo(lhs, rhs, bias, tiles))


def test_per_op_conv_matches_oracle(device, oracle_mod):
    rng = np.random.default_rng(22)
    x = rng.standard_normal((2, 3, 11, 13), dtype=np.float32)
    w = rng.standard_normal((4, 3, 3, 2), dtype=np.float32)
    b = rng.standard_normal(4, dtype=np.float32)
    stride, dil, pads, tiles = (2, 1), (1, 2), (1, 2, 0, 3), (3, 2, 1, 4, 5)
    ho, wo = oracle_mod.conv2d_out_hw(11, 13, 3, 2, stride, dil, pads)
    out = np.zeros((2, 4, ho, wo), np.float32)
    r = _run(conv2d_inputs_dynamic_tile_dynamic_kernel, (out, x, w, b, *stride, *dil, *pads, *tiles), PER_OP)
    assert r.fused is None
    assert np.array_equal(out, oracle_mod.conv2d_demo(x, w, b, stride, dil, pads, tiles))


@pytest.mark.parametrize("kernel_fn,causal", [(flash_attention_scaled_kernel, False),
                                              (flash_attention_scaled_causal_kernel, True)])
def test_per_op_attention_matches_oracle(device, oracle_mod, kernel_fn, causal):
    """exp and division in double on both sides: equal up to the last bit of the double
    exp the GPU library and glibc each round (checked at 2 ulp of fp32)."""

    rng = np.random.default_rng(23)
    q, k, v = (rng.standard_normal((1, 2, 45, 12), dtype=np.float32) for _ in range(3))
    out = np.zeros_like(q)
    r = _run(kernel_fn, (out, q, k, v, 12, 5, 0.29), PER_OP)
    assert r.fused is None
    ref = oracle_mod.flash_attention_demo(q, k, v, 12, 5, scale=0.29, causal=causal)
    ulp = np.spacing(np.abs(ref).astype(np.float32))
    assert np.all(np.abs(out - ref) <= 2 * ulp), np.max(np.abs(out - ref) / ulp)


def test_fused_and_per_op_paths_agree_on_16bit_attention(device, oracle_mod):
    """bf16 D=128: the fused path runs the MFMA kernel, the per-operation path the demo's
    loop nest in fp32 on the same rounded inputs; both meet the bf16 bar against the
    oracle."""

    import torch

    rng = np.random.default_rng(24)
    shape = (1, 2, 128, 128)
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), torch.bfloat16) for _ in range(3))
    outs = {}
    for name, options in (("fused", None), ("per-op", PER_OP)):
        out = torch.zeros(shape, dtype=torch.bfloat16, device="cuda")
        r = _run(flash_attention_scaled_causal_kernel, (out, qt.cuda(), kt.cuda(), vt.cuda(), 64, 32, 1 / np.sqrt(128)),
                 options)
        assert (r.fused is not None) == (name == "fused")
        outs[name] = to_numpy(out)
    ref = oracle_mod.flash_attention_demo(q, k, v, 64, 32, scale=1 / np.sqrt(128), causal=True)
    for name, got in outs.items():
        assert_h16_close(got, ref, what=name)


def test_renamed_kernel_runs_fused(device, oracle_mod):
    """A kernel with another name and other parameter names whose IR is the matmul nest
    is recognised and runs on the MFMA/fp32 GEMM kernels."""

    rng = np.random.default_rng(25)
    a = rng.standard_normal((130, 96), dtype=np.float32)
    b = rng.standard_normal((96, 70), dtype=np.float32)
    bias = rng.standard_normal(70, dtype=np.float32)
    c = np.zeros((130, 70), np.float32)
    r = _run(my_gemm, (c, a, b, bias, 32, 16, 8))
    assert r.fused is not None and r.fused.family == "matmul" and "kg_gfx950_matmul_entry" in r.source
    ref = oracle_mod.matmul_demo(a, b, bias, (32, 16, 8))
    assert np.allclose(c, ref, rtol=1e-4, atol=1e-4)


def softmax_rows_kernel(out: "Tensor[f32, R, C]", x: "Tensor[f32, R, C]", tile_r: SymbolDim) -> None:
    """Row softmax in tiles of rows: no hand-written kernel has this shape, so it runs on
    the per-operation path."""

    rows, cols = x.get_shape()
    for r0 in loop(0, rows, tile_r):
        cur = min(tile_r, rows - r0)
        t = alloc([cur, cols], NumericType.Float32, MemorySpace.TSM)
        deslice(t, view(x, [r0, 0], [cur, cols], [1, 1]), [0, 0], [cur, cols], [1, 1])
        mx = alloc([cur, 1], NumericType.Float32, MemorySpace.TSM)
        dsl_kernel.reduce(mx, t, kind=dsl_kernel.KernelReduceKind.MAX, axis=1, keepdim=True)
        full = alloc([cur, cols], NumericType.Float32, MemorySpace.TSM)
        broadcast(full, mx)
        dsl_kernel.sub(t, t, full)
        dsl_kernel.exp(t, t)
        sm = alloc([cur, 1], NumericType.Float32, MemorySpace.TSM)
        dsl_kernel.reduce(sm, t, kind=dsl_kernel.KernelReduceKind.SUM, axis=1, keepdim=True)
        broadcast(full, sm)
        dsl_kernel.truediv(t, t, full)
        deslice(out, t, [r0, 0], [cur, cols], [1, 1])


def test_unrecognised_kernel_runs_per_op(device):
    rng = np.random.default_rng(26)
    x = rng.standard_normal((37, 29), dtype=np.float32)
    out = np.zeros_like(x)
    r = _run(softmax_rows_kernel, (out, x, 8))
    assert r.fused is None
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    np.testing.assert_allclose(out, e / e.sum(1, keepdims=True), rtol=1e-5, atol=1e-6)
