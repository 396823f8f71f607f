"""memory_stage on every fused family: gfx950-lowering{memory_stage=N} sets the LDS ring
depth of the kernel a fused call selects (the reference's MultiBufferAnalysisPass option,
kernel_gen/passes/memory/multi_buffer.py:2071-2135,2281-2356): attention's K/V rings, the
fp32 GEMM's operand ring, the row-piece and implicit-GEMM conv kernels' stage count. A
deeper ring changes when copies land, never the order of any accumulation, so every depth
must give the default call's bits. A kernel the call selects that cannot take a ring depth
fails with an error that names it."""

from __future__ import annotations

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.gpu_util import assert_f32_close, assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu

ATTENTION = [
    ((1, 2, 256, 128), False, "bfloat16"),   # small grid: the 4-wave D=128 variant
    ((2, 16, 512, 128), False, "bfloat16"),  # the 8-wave variant
    ((1, 4, 300, 64), True, "bfloat16"),     # ragged causal D=64
    ((1, 3, 200, 128), True, "float16"),     # ragged causal D=128
]


@pytest.mark.parametrize("shape,causal,dtype", ATTENTION)
def test_attention_ring_depths_bit_identical(device, oracle_mod, shape, causal, dtype):
    import torch

    tdt = getattr(torch, dtype)
    rng = np.random.default_rng(sum(shape))
    q, k, v = (round_to(rng.standard_normal(shape, dtype=np.float32), tdt)[0].to(device) for _ in range(3))
    scale = 1.0 / np.sqrt(shape[3])
    default = torch.full(shape, float("nan"), dtype=tdt, device=device)
    native.flash_attention(default, q, k, v, 64, 64, scale, causal)
    for stages in (2, 3, 4):
        out = torch.full(shape, float("nan"), dtype=tdt, device=device)
        print(f"[attention] {shape} causal={causal} {dtype} memory_stage={stages}", flush=True)
        native.flash_attention(out, q, k, v, 64, 64, scale, causal, memory_stage=stages)
        assert torch.equal(out, default), f"memory_stage={stages}"
    ref = oracle_mod.flash_attention_demo(to_numpy(q[:1, :1]), to_numpy(k[:1, :1]), to_numpy(v[:1, :1]), 64, 64,
                                          scale=scale, causal=causal)
    assert_h16_close(to_numpy(default[:1, :1]), ref, what=f"{shape} head 0")


CONVS = [
    # (x shape, w shape, stride, pads, dtype): C3's geometry takes the row-piece kernel when staged
    ((2, 64, 16, 16), (64, 64, 3, 3), (1, 1), (1, 1, 1, 1), "float16"),
    ((2, 32, 28, 28), (64, 32, 3, 3), (2, 2), (1, 1, 1, 1), "bfloat16"),  # row-piece, stride 2
    ((2, 64, 14, 14), (32, 64, 1, 1), (1, 1), (0, 0, 0, 0), "float16"),   # row-piece 1x1
    ((2, 12, 21, 19), (24, 12, 5, 5), (2, 3), (2, 1, 0, 2), "bfloat16"),  # implicit GEMM
    ((2, 16, 28, 28), (32, 16, 3, 3), (1, 1), (1, 1, 1, 1), "float32"),   # fp32 row-piece
    ((1, 6, 17, 23), (10, 6, 3, 2), (1, 2), (0, 1, 1, 0), "float32"),     # fp32 implicit GEMM
]


@pytest.mark.parametrize("xs,ws,stride,pads,dtype", CONVS)
def test_conv_stage_counts_bit_identical(device, oracle_mod, xs, ws, stride, pads, dtype):
    import torch

    tdt = getattr(torch, dtype)
    rng = np.random.default_rng(sum(xs) + sum(ws))
    x = round_to(rng.standard_normal(xs, dtype=np.float32), tdt)[0].to(device)
    w = round_to(rng.uniform(-0.2, 0.2, ws).astype(np.float32), tdt)[0].to(device)
    ho, wo = oracle_mod.conv2d_out_hw(xs[2], xs[3], ws[2], ws[3], stride, (1, 1), pads)
    outs = []
    for stages in (2, 3, 4):
        out = torch.full((xs[0], ws[0], ho, wo), float("nan"), dtype=tdt, device=device)
        print(f"[conv2d] {xs} {ws} stride {stride} {dtype} memory_stage={stages}", flush=True)
        native.conv2d(out, x, w, None, stride, (1, 1), pads, memory_stage=stages)
        outs.append(out)
    for stages, out in zip((3, 4), outs[1:]):
        assert torch.equal(out, outs[0]), f"memory_stage={stages}"
    ref = oracle_mod.conv2d_demo(to_numpy(x), to_numpy(w), None, stride, (1, 1), pads, (8, 8, 1, 8, 8))
    if dtype == "float32":
        assert_f32_close(to_numpy(outs[0]), ref, rtol=1e-4, atol=1e-4 * max(1.0, float(np.abs(ref).max())),
                         what="staged fp32 conv")
    else:
        assert_h16_close(to_numpy(outs[0]), ref, what="staged 16-bit conv")


def test_fp32_gemm_ring_depths_bit_identical(device, oracle_mod):
    import torch

    m, n, k = 1024, 768, 560  # 48 tiles of 128 x 128: the fp32 MFMA kernel; K = 35 slices of 16
    rng = np.random.default_rng(3)
    a = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to(device)
    b = torch.from_numpy(rng.standard_normal((k, n), dtype=np.float32)).to(device)
    default = torch.full((m, n), float("nan"), device=device)
    native.matmul(default, a, b, None)
    for stages in (2, 3, 4):
        out = torch.full((m, n), float("nan"), device=device)
        print(f"[matmul f32] memory_stage={stages}", flush=True)
        native.call_entry("kg_gfx950_matmul_entry", (out, a, b, None, 64, 64, 64, stages))
        assert torch.equal(out, default), f"memory_stage={stages}"
    ref = oracle_mod.matmul_demo(a[:64].cpu().numpy(), b.cpu().numpy(), None, (64, 64, 64))
    assert_f32_close(to_numpy(default[:64]), ref, rtol=1e-4, atol=4 * np.sqrt(k) * 2.0 ** -24 * 64, what="rows 0:64")


def test_kernels_without_a_ring_reject_memory_stage(device):
    import torch

    dev = device
    # fp32 attention on the fp32 MFMA kernel: two fixed K and V buffers
    x = torch.randn(1, 2, 128, 64, device=dev)
    o = torch.empty_like(x)
    with pytest.raises(native.NativeLibraryError, match="two K and two V buffers"):
        native.flash_attention(o, x, x, x, 64, 64, 0.125, False, memory_stage=3)
    native.flash_attention(o, x, x, x, 64, 64, 0.125, False, memory_stage=2)  # its own depth is accepted
    # attention on the SIMT kernel (head dim 48)
    y = torch.randn(1, 2, 64, 48, device=dev)
    with pytest.raises(native.NativeLibraryError, match="SIMT kernel"):
        native.flash_attention(torch.empty_like(y), y, y, y, 64, 64, 0.125, False, memory_stage=2)
    # a 16-bit matmul with K % 8 != 0 takes the SIMT GEMM
    a = torch.randn(64, 36, device=dev).to(torch.bfloat16)
    b = torch.randn(36, 64, device=dev).to(torch.bfloat16)
    with pytest.raises(native.NativeLibraryError, match="SIMT kernel"):
        native.call_entry("kg_gfx950_matmul_entry", (torch.empty(64, 64, device=dev, dtype=torch.bfloat16), a, b, None,
                                                     8, 8, 8, 3))
    # a conv whose output is not 16-byte aligned takes the direct kernel
    xs = torch.randn(1, 4, 8, 8, device=dev)
    ws = torch.randn(4, 4, 3, 3, device=dev)
    flat = torch.empty(4 * 8 * 8 + 1, device=dev)
    out = flat[1:].view(1, 4, 8, 8)
    with pytest.raises(native.NativeLibraryError, match="direct kernel"):
        native.conv2d(out, xs, ws, None, (1, 1), (1, 1), (1, 1, 1, 1), memory_stage=2)
