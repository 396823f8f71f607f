"""GPU parity of the gfx950 conv2d entry (kg_gfx950_conv2d_entry) against the CPU oracle.

Cases follow the reference's runtime test (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:
530-566: arange inputs, arange/7 weights, stride 8, asymmetric pads), the conv2d demos'
random static/dynamic shapes (kernel/conv2d/*.py) and BASELINE config C3 (fp16 NCHW
32x64x56x56, 64 filters 3x3, stride 1, pad 1).
"""

from __future__ import annotations

import random
from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.golden.make_golden import BIG_CONV_CASE, conv_closed_form
from tests.gpu_util import assert_f32_close, assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def out_hw(xs, ws, stride, dil, pad):
    ho = (xs[2] + pad[0] + pad[1] - dil[0] * (ws[2] - 1) - 1) // stride[0] + 1
    wo = (xs[3] + pad[2] + pad[3] - dil[1] * (ws[3] - 1) - 1) // stride[1] + 1
    return ho, wo


def run(device, dtype, x, w, bias, stride, dil, pad, tiles=()):
    import torch

    xt = torch.as_tensor(x).to(device)
    wt = torch.as_tensor(w).to(device)
    bt = None if bias is None else torch.as_tensor(bias).to(device)
    ho, wo = out_hw(xt.shape, wt.shape, stride, dil, pad)
    out = torch.full((xt.shape[0], wt.shape[0], ho, wo), float("nan"), dtype=dtype, device=device)
    print(f"[conv2d] x={tuple(xt.shape)} w={tuple(wt.shape)} s={stride} d={dil} p={pad} {dtype}", flush=True)
    native.conv2d(out, xt, wt, bt, stride, dil, pad, tiles)
    return out


@pytest.mark.parametrize("case", [0, 1])
def test_runtime_vectors(device, case):
    import torch

    v = dict(np.load(GOLDEN / "cuda_runtime_vectors.npz"))
    p = v[f"conv{case}_params"]
    xs, ws, stride, dil, pad = tuple(p[0:4]), tuple(p[4:8]), tuple(p[8:10]), tuple(p[10:12]), tuple(p[12:16])
    x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs)
    w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
    b = np.arange(ws[0], dtype=np.float32)
    tiles = (7, 18, 3, 9, 8)
    assert_f32_close(to_numpy(run(device, torch.float32, x, w, None, stride, dil, pad, tiles)), v[f"conv{case}_absent"],
                     rtol=1e-5, atol=1e-5, what="absent")
    assert_f32_close(to_numpy(run(device, torch.float32, x, w, b, stride, dil, pad, tiles)), v[f"conv{case}_present"],
                     rtol=1e-5, atol=1e-5, what="present")


def test_runtime_big_static_case(device, oracle_mod):
    # (4,49,248,232) x (20,49,3,5), stride 8, pads (3,3,4,0): the reference's first conv case
    import torch

    xs, ws, stride, dil, pad = BIG_CONV_CASE
    x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs) / np.float32(1e6)
    w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
    b = np.arange(ws[0], dtype=np.float32)
    ref = oracle_mod.conv2d_demo(x, w, b, stride, dil, pad, (8, 16, 4, 8, 9))
    assert_f32_close(to_numpy(run(device, torch.float32, x, w, b, stride, dil, pad)), ref, what="big static")


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_demo_random_profiles_f32(device, oracle_mod, seed):
    """Shapes drawn like kernel/conv2d/inputs_static_tile_static.py:283-300 (stride 8)."""

    import torch

    r = random.Random(seed)
    n, c = r.randint(1, 2), r.randint(8, 16)
    h, w = r.randint(41, 89), r.randint(25, 73)
    f = r.randint(18, 24)
    kh, kw = r.choice((3, 5)), r.choice((3, 5))
    pad = tuple(r.choice((0, 1, 2, 3, 4)) for _ in range(4))
    tiles = r.choice(((8, 16, 4, 8, 9), (7, 18, 3, 9, 8), (6, 20, 2, 10, 7)))
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, c, h, w)).astype(np.float32)
    wt = rng.normal(size=(f, c, kh, kw)).astype(np.float32)
    b = rng.normal(size=(f,)).astype(np.float32)
    ref = oracle_mod.conv2d_demo(x, wt, b, (8, 8), (1, 1), pad, tiles)
    assert_f32_close(to_numpy(run(device, torch.float32, x, wt, b, (8, 8), (1, 1), pad, tiles)), ref, what=str(seed))


@pytest.mark.parametrize(
    "xs,ws,stride,dil,pad",
    [
        ((2, 5, 17, 19), (4, 5, 3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
        ((1, 3, 20, 21), (6, 3, 2, 3), (2, 3), (2, 1), (0, 4, 2, 1)),
        ((1, 2, 4, 5), (3, 2, 2, 2), (1, 1), (1, 1), (1, 1, 1, 1)),
    ],
)
def test_general_params_f32(device, oracle_mod, xs, ws, stride, dil, pad):
    import torch

    rng = np.random.default_rng(sum(xs))
    x = rng.normal(size=xs).astype(np.float32)
    w = rng.normal(size=ws).astype(np.float32)
    for b in (None, rng.normal(size=(ws[0],)).astype(np.float32)):
        ref = oracle_mod.conv2d_demo(x, w, b, stride, dil, pad, (8, 16, 4, 8, 9))
        assert_f32_close(to_numpy(run(device, torch.float32, x, w, b, stride, dil, pad)), ref, what=str(xs))


@pytest.mark.parametrize("dtype_name", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize(
    "xs,ws,stride,dil,pad,bias",
    [
        ((2, 64, 56, 56), (64, 64, 3, 3), (2, 2), (1, 1), (1, 1, 1, 1), None),  # stride 2
        ((2, 128, 28, 28), (128, 128, 3, 3), (1, 1), (1, 1), (1, 1, 1, 1), "f32"),  # 128-filter tiles
        ((4, 256, 14, 14), (256, 256, 1, 1), (1, 1), (1, 1), (0, 0, 0, 0), None),  # 1x1
        ((2, 3, 64, 64), (64, 3, 7, 7), (2, 2), (1, 1), (3, 3, 3, 3), "same"),  # K = 147: scalar weights
        ((1, 40, 19, 23), (96, 40, 3, 3), (1, 2), (2, 1), (2, 1, 0, 3), "f32"),  # F = 96, Ho*Wo odd
        ((3, 24, 10, 10), (20, 24, 5, 5), (1, 1), (2, 2), (4, 4, 4, 4), None),  # dilated, F < 32
        ((2, 512, 7, 7), (512, 512, 3, 3), (1, 1), (1, 1), (1, 1, 1, 1), "f32"),  # 8 tiles: K split 36-58 ways
        ((2, 256, 14, 14), (256, 256, 3, 3), (2, 2), (1, 1), (1, 1, 1, 1), "same"),  # stride 2, K split
    ],
    ids=["s2", "c128", "1x1", "7x7s2", "f96_ragged", "dilated", "7x7_c512_splitk", "14x14s2_splitk"],
)
def test_implicit_gemm_shapes(device, oracle_mod, dtype_name, xs, ws, stride, dil, pad, bias):
    """Every conv the 3x3 kernel does not take runs as an implicit GEMM on matrix cores (16-bit
    or fp32 MFMA); grids of fewer than two workgroups per CU split K into fp32 partials added in
    a fixed order (the 1x1, ragged, dilated and the last two cases). Reference: the oracle's
    demo loop nest on the identically rounded inputs.
    fp32 tolerance: the demo's rtol 1e-4 / atol 1e-5 plus the rounding that two fp32 summation
    orders of K = C KH KW products can differ by, 4 sqrt(K) 2^-24 (|W| * |X|) (the
    probabilistic bound of Higham and Mary, SIAM J. Sci. Comput. 41 (2019))."""

    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(sum(xs) + sum(ws))
    k = ws[1] * ws[2] * ws[3]
    bound = np.sqrt(6.0 / k)
    if dt == torch.float32:
        x = rng.standard_normal(xs).astype(np.float32)
        w = rng.uniform(-bound, bound, size=ws).astype(np.float32)
        xt, wt = torch.from_numpy(x), torch.from_numpy(w)
    else:
        xt, x = round_to(rng.standard_normal(xs), dt)
        wt, w = round_to(rng.uniform(-bound, bound, size=ws), dt)
    b = bt = None
    if bias == "f32":
        b = bt = rng.normal(size=(ws[0],)).astype(np.float32)
    elif bias == "same":
        if dt == torch.float32:
            b = bt = rng.normal(size=(ws[0],)).astype(np.float32)
        else:
            bt, b = round_to(rng.normal(size=(ws[0],)).astype(np.float32), dt)
    tiles = (16, 16, 1, 8, 16)
    ref = oracle_mod.conv2d_demo(x, w, b, stride, dil, pad, tiles)
    out = to_numpy(run(device, dt, xt, wt, bt, stride, dil, pad))
    what = f"{dtype_name} {xs} {ws} s={stride} d={dil} p={pad} bias={bias}"
    if dt == torch.float32:
        terms = oracle_mod.conv2d_demo(np.abs(x), np.abs(w), None, stride, dil, pad, tiles).astype(np.float64)
        tol = 1e-4 * np.abs(ref) + 1e-5 + 4 * np.sqrt(k) * 2.0 ** -24 * terms
        err = np.abs(out.astype(np.float64) - ref)
        assert (err <= tol).all(), f"{what}: max err/tol {np.max(err / tol):.3g}"
    else:
        assert_h16_close(out, ref, what=what)


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
@pytest.mark.parametrize(
    "xs,ws,bias",
    [
        ((2, 64, 56, 56), (64, 64, 3, 3), None),  # C3 geometry, 2 images (MFMA path)
        ((1, 64, 12, 24), (64, 64, 3, 3), "f32"),  # MFMA: 7-row blocks with a 5-row tail, W <= 32
        ((3, 64, 20, 40), (64, 64, 3, 3), "h16"),  # MFMA: 6-row tail, second pixel block partly live
        ((1, 64, 1, 8), (64, 64, 3, 3), "f32"),  # MFMA: one row, one 8-column block
        ((2, 64, 9, 32), (64, 64, 3, 3), "h16"),  # MFMA: second window live for pixels 28-31 only
        ((1, 64, 15, 48), (64, 64, 3, 3), None),  # MFMA: 1-row tail, second window partly live
        ((1, 64, 12, 20), (64, 64, 3, 3), "f32"),  # W % 8 != 0: implicit GEMM on 4-pixel row pieces
        ((3, 16, 9, 13), (32, 16, 3, 3), "f32"),
        ((1, 8, 7, 7), (5, 8, 3, 3), None),
    ],
)
def test_16bit_3x3(device, oracle_mod, dtype_name, xs, ws, bias):
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(xs[1] + ws[0] + xs[2])
    xt, x = round_to(rng.standard_normal(xs), dt)
    bound = np.sqrt(6.0 / (ws[1] * 9))
    wt, w = round_to(rng.uniform(-bound, bound, size=ws), dt)
    b = bt = None
    if bias == "f32":
        b = bt = rng.normal(size=(ws[0],)).astype(np.float32)
    elif bias == "h16":  # bias in the output format
        bt, b = round_to(rng.normal(size=(ws[0],)).astype(np.float32), dt)
    ref = oracle_mod.conv2d_demo(x, w, b, (1, 1), (1, 1), (1, 1, 1, 1), (16, 16, 1, 8, 16))
    out = run(device, dt, xt, wt, bt, (1, 1), (1, 1), (1, 1, 1, 1))
    assert_h16_close(to_numpy(out), ref, what=f"{dtype_name} {xs} bias={bias}")


def _rowvec_mfma(xs, ws, stride, pad, f32=False):
    """MFMA instructions of the row-piece implicit GEMM (128-pixel tiles, 4 waves x MI x 2
    blocks, MI = 2 for F > 64 with >= 512 workgroups; 16-bit: 16-run K slices of KW
    32x32x16 steps, fp32: 8-run slices of 4 KW 32x32x2 MFMAs)."""

    n, c, h, w = xs
    f, _, kh, kw = ws
    ho, wo = out_hw(xs, ws, stride, (1, 1), pad)
    cols = -(-(n * ho * wo) // 128)
    mi = 2 if f > 64 and -(-f // 128) * cols >= 512 else 1
    runs, per = (8, 4) if f32 else (16, 1)
    return -(-f // (64 * mi)) * cols * -(-(c * kh) // runs) * 4 * mi * 2 * kw * per


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize(
    "xs,ws,stride,pad,bias,images",
    [
        ((2, 48, 16, 64), (64, 48, 3, 3), 1, (1, 1, 1, 1), "f32", None),  # 8-pixel pieces
        ((2, 40, 12, 28), (80, 40, 3, 3), 1, (1, 1, 1, 1), "same", None),  # 4-pixel pieces, F = 80, K slices ragged
        ((1, 16, 9, 24), (32, 16, 5, 3), 1, (2, 2, 1, 1), None, None),  # KH = 5
        ((2, 24, 10, 16), (48, 24, 3, 3), 1, (0, 2, 1, 1), "f32", None),  # asymmetric vertical pads
        ((2, 32, 6, 28), (40, 32, 1, 1), 1, (0, 0, 0, 4), "same", None),  # 1x1, right pad: Wo = 32 > W
        ((16, 32, 64, 64), (128, 32, 3, 3), 1, (1, 1, 1, 1), "f32", (0, 15)),  # 128-filter tiles
        ((2, 64, 56, 56), (128, 64, 3, 3), 2, (1, 1, 1, 1), None, None),  # stride 2, Wo = 28: 4-pixel pieces
        ((1, 24, 17, 32), (40, 24, 3, 3), 2, (1, 0, 1, 1), "f32", None),  # stride 2, odd H, 8-pixel pieces
        ((2, 32, 32, 64), (64, 32, 1, 1), 2, (0, 0, 0, 0), "same", None),  # 1x1 stride 2
        ((1, 16, 8, 40), (24, 16, 1, 1), 2, (0, 0, 0, 0), None, None),  # 1x1 stride 2, Wo = 20
        ((1, 120, 28, 28), (96, 120, 3, 3), 1, (1, 1, 1, 1), "same", None),  # 7 workgroups: K split, last chunk short
        ((1, 256, 8, 32), (64, 256, 1, 1), 1, (0, 0, 0, 0), "f32", None),  # 1x1, 2 workgroups: K split
    ],
    ids=["p8", "p4_f80", "kh5", "pads_0_2", "1x1_rpad", "bm128", "s2_p4", "s2_p8", "1x1_s2", "1x1_s2_p4",
         "splitk", "1x1_splitk"],
)
def test_row_piece_path(device, oracle_mod, dtype_name, xs, ws, stride, pad, bias, images):
    """Convs of stride 1 or 2 whose rows split into whole 8- or 4-pixel pieces (fp32: 4), with
    a 3-wide window and left pad 1 or a 1-wide window and left pad 0: each thread loads
    aligned row pieces once for all taps of a (c, kh) run and builds the windows in
    registers. The entry's cost query must count this kernel's MFMAs (so the case runs the
    row-piece path); output against the oracle on the identically rounded inputs (`images`:
    the images checked, the rest of the batch only runs). fp32 bar: rtol 1e-4 / atol 1e-5
    plus 4 sqrt(K) 2^-24 (|W| * |X|), the summation-order bound used for the implicit GEMM."""

    import torch

    dt = getattr(torch, dtype_name)
    f32 = dt == torch.float32
    st = (stride, stride)
    rng = np.random.default_rng(sum(xs) + sum(ws) + sum(pad) + stride)
    k = ws[1] * ws[2] * ws[3]
    bound = np.sqrt(6.0 / k)
    if f32:
        x = rng.standard_normal(xs).astype(np.float32)
        w = rng.uniform(-bound, bound, size=ws).astype(np.float32)
        xt, wt = torch.from_numpy(x), torch.from_numpy(w)
    else:
        xt, x = round_to(rng.standard_normal(xs), dt)
        wt, w = round_to(rng.uniform(-bound, bound, size=ws), dt)
    b = bt = None
    if bias == "f32" or (bias == "same" and f32):
        b = bt = rng.normal(size=(ws[0],)).astype(np.float32)
    elif bias == "same":
        bt, b = round_to(rng.normal(size=(ws[0],)).astype(np.float32), dt)
    ho, wo = out_hw(xs, ws, st, (1, 1), pad)
    spec = [native.TensorSpec((xs[0], ws[0], ho, wo), dtype_name), native.TensorSpec(xs, dtype_name),
            native.TensorSpec(ws, dtype_name),
            None if bt is None else native.TensorSpec((ws[0],), "float32" if bias == "f32" else dtype_name),
            stride, stride, 1, 1, *pad]
    assert native.cost("conv2d", spec)["MFMA"] == _rowvec_mfma(xs, ws, st, pad, f32)
    out = to_numpy(run(device, dt, xt, wt, bt, st, (1, 1), pad))
    assert np.isfinite(out).all()
    sel = slice(None) if images is None else list(images)
    tiles = (16, 16, 1, 8, 16)
    ref = oracle_mod.conv2d_demo(x[sel], w, b, st, (1, 1), pad, tiles)
    what = f"{dtype_name} {xs} {ws} s={stride} p={pad} bias={bias}"
    if f32:
        terms = oracle_mod.conv2d_demo(np.abs(x[sel]), np.abs(w), None, st, (1, 1), pad, tiles).astype(np.float64)
        tol = 1e-4 * np.abs(ref) + 1e-5 + 4 * np.sqrt(k) * 2.0 ** -24 * terms
        err = np.abs(out[sel].astype(np.float64) - ref)
        assert (err <= tol).all(), f"{what}: max err/tol {np.max(err / tol):.3g}"
    else:
        assert_h16_close(out[sel], ref, what=what)


def test_c3_full_size_fp16(device, oracle_mod):
    """BASELINE C3 at full size: two images against the oracle, the whole batch against
    per-image linearity (conv(x_a + x_b) = conv(x_a) + conv(x_b)) in fp32 math."""

    import torch

    rng = np.random.default_rng(20261204)
    xt, x = round_to(rng.standard_normal((32, 64, 56, 56), dtype=np.float32), torch.float16)
    bound = np.sqrt(6.0 / 576.0)
    wt, w = round_to(rng.uniform(-bound, bound, size=(64, 64, 3, 3)).astype(np.float32), torch.float16)
    out = to_numpy(run(device, torch.float16, xt, wt, None, (1, 1), (1, 1), (1, 1, 1, 1)))
    for i in (0, 31):
        ref = oracle_mod.conv2d_demo(x[i : i + 1], w, None, (1, 1), (1, 1), (1, 1, 1, 1), (16, 16, 1, 8, 16))
        assert_h16_close(out[i : i + 1], ref, what=f"C3 image {i}")
    # batch consistency: image i of the batched call equals a single-image call
    single = to_numpy(run(device, torch.float16, xt[17:18], wt, None, (1, 1), (1, 1), (1, 1, 1, 1)))
    np.testing.assert_array_equal(single, out[17:18])
    closed = conv_closed_form(x[5:6], w, None, (1, 1), (1, 1), (1, 1, 1, 1))
    assert_h16_close(out[5:6], closed, what="C3 closed form image 5")


def test_rejects_bad_params(device):
    import torch

    x = torch.zeros(1, 2, 5, 5, device=device)
    w = torch.zeros(3, 2, 3, 3, device=device)
    o = torch.zeros(1, 3, 5, 5, device=device)
    with pytest.raises(native.NativeLibraryError):
        native.conv2d(o, x, w, None, (0, 1), (1, 1), (1, 1, 1, 1))
    with pytest.raises(native.NativeLibraryError):
        native.conv2d(o, x, w, None, (1, 1), (1, 1), (0, 0, 0, 0))  # out shape mismatch
