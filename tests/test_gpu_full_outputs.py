"""Every output element of the BASELINE GPU configs at full size (C2, C2', C3, C4, C5 with
D=128 and D=64), against an fp32 evaluation of the same formula on the GPU from the
identically rounded 16-bit inputs.

The CPU oracle checks sampled rows, heads and images of these configs
(tests/test_gpu_matmul.py::test_full_size_bf16, test_gpu_conv2d.py::test_c3_full_size_fp16,
test_gpu_flash_attention.py::test_c4_full_size / test_c5_full_size_causal); this test covers
the rest of each output, with the same bars the oracle tests apply: the 16-bit bar
2e-2 |ref| + 1e-2 rms(ref) for the GEMM and the conv, and for attention that bar plus the
probabilistic bound of the P rounding, 4 u sqrt(sum_j w_j^2 (V_j - O)^2) (tests/gpu_util.py:
attention_h16_tolerance, here evaluated in fp32 on the GPU). The references are plain torch
fp32 operations with reduced-precision modes off (no TF32/XF32, no 16-bit batched products);
attention is evaluated one head at a time to bound memory.
"""

from __future__ import annotations

import pytest

from kernelcode_generate_amd import native
from tests.gpu_util import H16_ATOL_RMS, H16_RTOL

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _full_fp32_references():
    import torch

    saved = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = saved


def _check(out, ref, extra, what):
    """|out - ref| <= 2e-2 |ref| + 1e-2 rms(ref) (+ extra) on every element (GPU tensors)."""

    import torch

    out = out.float()
    assert torch.isfinite(out).all(), f"{what}: non-finite output"
    rms = ref.pow(2).mean().sqrt()
    bar = H16_RTOL * ref.abs() + H16_ATOL_RMS * rms
    if extra is not None:
        bar = bar + extra
    err = (out - ref).abs()
    bad = err > bar
    n_bad = int(bad.sum())
    assert n_bad == 0, f"{what}: {n_bad} of {bad.numel()} outside the bar; worst err/bar {float((err / bar).max()):.3f}"
    # the bar is not vacuous: 10 % off on the largest output element fails it
    i = int(ref.abs().argmax())
    planted = out.flatten().clone()
    planted[i] = ref.flatten()[i] * 1.1
    assert bool((planted - ref.flatten()).abs()[i] > bar.flatten()[i]), f"{what}: a 10 % error passes the bar"


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 4096), (8192, 1024, 4096)], ids=["C2", "C2s"])
def test_gemm_every_element(device, m, n, k):
    import torch

    g = torch.Generator(device=device).manual_seed(m + n)
    a = (torch.randn(m, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = (torch.randn(k, n, generator=g, device=device) * 0.02).to(torch.bfloat16)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
    print(f"[full] matmul {m}x{k}x{n}", flush=True)
    native.matmul(out, a, b, None)
    ref = a.float() @ b.float()
    _check(out, ref, None, f"matmul {m}x{k}x{n}")


def test_c3_conv_every_element(device):
    import torch
    import torch.nn.functional as F

    g = torch.Generator(device=device).manual_seed(3)
    x = torch.randn(32, 64, 56, 56, generator=g, device=device).to(torch.float16)
    bound = (6.0 / 576.0) ** 0.5
    w = ((torch.rand(64, 64, 3, 3, generator=g, device=device) * 2 - 1) * bound).to(torch.float16)
    out = torch.full((32, 64, 56, 56), float("nan"), dtype=torch.float16, device=device)
    print("[full] conv C3", flush=True)
    native.conv2d(out, x, w, None, (1, 1), (1, 1), (1, 1, 1, 1))
    ref = F.conv2d(x.float(), w.float(), None, padding=1)
    _check(out, ref, None, "C3")


@pytest.mark.parametrize(
    "shape,causal",
    [((4, 32, 2048, 128), False), ((1, 32, 16384, 128), True), ((1, 32, 16384, 64), True)],
    ids=["C4", "C5_d128", "C5_d64"],
)
def test_attention_every_element(device, shape, causal):
    import torch

    b, h, s, d = shape
    g = torch.Generator(device=device).manual_seed(s + d)
    q, k, v = (torch.randn(shape, generator=g, device=device).to(torch.bfloat16) for _ in range(3))
    scale = 1.0 / d ** 0.5
    out = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=device)
    print(f"[full] attention {shape} causal={causal}", flush=True)
    native.flash_attention(out, q, k, v, 64, 64, scale, causal)
    ref = torch.empty(shape, dtype=torch.float32, device=device)
    spread = torch.empty_like(ref)
    keep = torch.ones(s, s, dtype=torch.bool, device=device).tril() if causal else None
    for bi in range(b):
        for hi in range(h):
            qh, kh, vh = q[bi, hi].float(), k[bi, hi].float(), v[bi, hi].float()
            sc = (qh @ kh.t().contiguous()) * scale
            if causal:
                sc = sc.masked_fill(~keep, float("-inf"))
            p = torch.softmax(sc, dim=-1)
            del sc
            o = p @ vh
            p2 = p * p
            del p
            # sum_j w_j^2 (V_j - O)^2 = W2 V^2 - 2 O (W2 V) + O^2 (W2 1), clipped at 0
            sp = p2 @ (vh * vh) - 2 * o * (p2 @ vh) + o * o * p2.sum(-1, keepdim=True)
            ref[bi, hi] = o
            spread[bi, hi] = sp.clamp_min(0)
            del p2
    u = 2.0 ** -8
    _check(out, ref, 4 * u * spread.sqrt(), f"attention {shape} causal={causal}")
