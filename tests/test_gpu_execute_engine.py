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
