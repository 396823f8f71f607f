"""Seeded random shapes through the 16-bit matmul, the conv (3x3 row-block kernel and the
row-piece implicit GEMM, 16-bit and fp32) and attention entries against the CPU oracle: many
small and ragged shapes in one place, including matmuls that take the split-K path (outputs of
at most 64 tiles with K >= 512), strided output windows and every bias form."""

from __future__ import annotations

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.gpu_util import assert_h16_close, assert_within, attention_h16_tolerance, round_to, to_numpy

pytestmark = pytest.mark.gpu


def _matmul_cases(n_cases=24, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n_cases):
        m = int(rng.choice([1, 3, 16, 31, 64, 100, 128, 129, 257, 300]))
        k = 8 * int(rng.integers(1, 257))  # 8 .. 2048
        n = 8 * int(rng.integers(1, 129))  # 8 .. 1024
        dt = "bfloat16" if i % 2 == 0 else "float16"
        bias = ["none", "f32", "same"][i % 3]
        pad = int(rng.integers(0, 2)) * 8  # extra output columns (strided window)
        cases.append((m, k, n, dt, bias, pad))
    return cases


@pytest.mark.parametrize("m,k,n,dtype_name,bias_kind,pad", _matmul_cases())
def test_random_matmul(device, oracle_mod, m, k, n, dtype_name, bias_kind, pad):
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(m * 1000003 + k * 1009 + n)
    lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.1, dt)
    rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.1, dt)
    bias = bt = None
    if bias_kind == "f32":
        bias = bt = rng.standard_normal(n).astype(np.float32)
    elif bias_kind == "same":
        bt, bias = round_to(rng.standard_normal(n), dt)
    big = torch.full((m + 1, n + pad), float("nan"), dtype=dt, device=device)
    out = big[:m, :n]
    print(f"[random] matmul M={m} K={k} N={n} {dtype_name} bias={bias_kind} ldc={n + pad}", flush=True)
    native.matmul(out, lt.to(device), rt.to(device), None if bt is None else torch.as_tensor(bt).to(device))
    got = to_numpy(big)
    assert np.isnan(got[m:]).all() and np.isnan(got[:, n:]).all(), "store outside the output window"
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, (64, 64, 64))
    assert_h16_close(got[:m, :n], ref, what=f"matmul {m}x{k}x{n} {dtype_name} bias={bias_kind}")


def _conv_cases(n_cases=8, seed=20261204):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 4)), int(rng.integers(1, 30)), 8 * int(rng.integers(1, 8)),
             "float16" if i % 2 == 0 else "bfloat16", ["none", "f32", "same"][i % 3]) for i in range(n_cases)]


@pytest.mark.parametrize("n,h,w,dtype_name,bias_kind", _conv_cases())
def test_random_conv3x3(device, oracle_mod, n, h, w, dtype_name, bias_kind):
    """C = F = 64, 3x3, stride 1, pad 1, W a multiple of 8 up to 56: the row-block MFMA kernel
    (row-block tails, one- and two-pixel-block rows)."""

    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(n * 10007 + h * 101 + w)
    xt, x = round_to(rng.standard_normal((n, 64, h, w), dtype=np.float32), dt)
    bound = np.sqrt(6.0 / 576)
    wt, wgt = round_to(rng.uniform(-bound, bound, size=(64, 64, 3, 3)).astype(np.float32), dt)
    bias = bt = None
    if bias_kind == "f32":
        bias = bt = rng.standard_normal(64).astype(np.float32)
    elif bias_kind == "same":
        bt, bias = round_to(rng.standard_normal(64), dt)
    out = torch.full((n, 64, h, w), float("nan"), dtype=dt, device=device)
    print(f"[random] conv N={n} H={h} W={w} {dtype_name} bias={bias_kind}", flush=True)
    native.conv2d(out, xt.to(device), wt.to(device), None if bt is None else torch.as_tensor(bt).to(device),
                  (1, 1), (1, 1), (1, 1, 1, 1))
    ref = oracle_mod.conv2d_demo(x, wgt, bias, (1, 1), (1, 1), (1, 1, 1, 1), (16, 16, 1, 8, 16))
    assert_h16_close(to_numpy(out), ref, what=f"conv {n}x64x{h}x{w} {dtype_name} bias={bias_kind}")


def _rowvec_cases(n_cases=16, seed=20261206):
    """Random convs the row-piece kernels take: stride 1 or 2, 3x3 (left pad 1) or 1x1 (pad 0),
    W a multiple of 8 or 4 with a matching Wo, random C, F, H, vertical pads, dtype."""

    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        i = len(cases)
        k = [3, 1][i % 2]
        stride = int(rng.integers(1, 3))
        c = 8 * int(rng.integers(1, 13))
        f = int(rng.integers(1, 150))
        h = int(rng.integers(1, 24))
        w = 4 * int(rng.integers(1, 25))
        pt, pb = (int(rng.integers(0, 3)), int(rng.integers(0, 3))) if k == 3 else (0, 0)
        pads = (pt, pb, 1, 1) if k == 3 else (0, 0, 0, 0)
        ho = (h + pt + pb - k) // stride + 1
        wo = (w + pads[2] + pads[3] - k) // stride + 1
        if ho < 1 or wo < 1 or wo % 4:
            continue
        dt = ["float16", "bfloat16", "float32"][i % 3]
        cases.append((int(rng.integers(1, 4)), c, h, w, f, k, stride, pads, dt, ["none", "f32", "same"][i % 3]))
    return cases


@pytest.mark.parametrize("n,c,h,w,f,k,stride,pads,dtype_name,bias_kind", _rowvec_cases())
def test_random_row_piece_conv(device, oracle_mod, n, c, h, w, f, k, stride, pads, dtype_name, bias_kind):
    """The row-piece implicit GEMM (8- or 4-pixel row pieces shared by all taps) on random
    shapes; the fp32 bar adds the summation-order bound 4 sqrt(K) 2^-24 (|W| * |X|)."""

    import torch

    dt = getattr(torch, dtype_name)
    f32 = dt == torch.float32
    rng = np.random.default_rng(n * 7 + c * 11 + h * 13 + w * 17 + f * 19 + k + stride)
    kk = c * k * k
    bound = np.sqrt(6.0 / kk)
    if f32:
        x = rng.standard_normal((n, c, h, w)).astype(np.float32)
        wgt = rng.uniform(-bound, bound, size=(f, c, k, k)).astype(np.float32)
        xt, wt = torch.from_numpy(x), torch.from_numpy(wgt)
    else:
        xt, x = round_to(rng.standard_normal((n, c, h, w), dtype=np.float32), dt)
        wt, wgt = round_to(rng.uniform(-bound, bound, size=(f, c, k, k)).astype(np.float32), dt)
    bias = bt = None
    if bias_kind == "f32" or (bias_kind == "same" and f32):
        bias = bt = rng.standard_normal(f).astype(np.float32)
    elif bias_kind == "same":
        bt, bias = round_to(rng.standard_normal(f), dt)
    ho = (h + pads[0] + pads[1] - k) // stride + 1
    wo = (w + pads[2] + pads[3] - k) // stride + 1
    out = torch.full((n, f, ho, wo), float("nan"), dtype=dt, device=device)
    st = (stride, stride)
    spec = [native.TensorSpec(tuple(out.shape), dtype_name), native.TensorSpec(tuple(xt.shape), dtype_name),
            native.TensorSpec(tuple(wt.shape), dtype_name), None, stride, stride, 1, 1, *pads]
    runs, per = (8, 4) if f32 else (16, 1)
    cols = -(-(n * ho * wo) // 128)
    mi = 2 if f > 64 and -(-f // 128) * cols >= 512 else 1
    assert native.cost("conv2d", spec)["MFMA"] == -(-f // (64 * mi)) * cols * -(-(c * k) // runs) * 8 * mi * k * per
    print(f"[random] row-piece conv N={n} C={c} H={h} W={w} F={f} {k}x{k} s{stride} p={pads} {dtype_name} "
          f"bias={bias_kind}", flush=True)
    native.conv2d(out, xt.to(device), wt.to(device), None if bt is None else torch.as_tensor(bt).to(device),
                  st, (1, 1), pads)
    got = to_numpy(out)
    tiles = (16, 16, 1, 8, 16)
    ref = oracle_mod.conv2d_demo(x, wgt, bias, st, (1, 1), pads, tiles)
    what = f"row-piece conv {n}x{c}x{h}x{w} F={f} {k}x{k} s{stride} p={pads} {dtype_name} bias={bias_kind}"
    if f32:
        terms = oracle_mod.conv2d_demo(np.abs(x), np.abs(wgt), None, st, (1, 1), pads, tiles).astype(np.float64)
        tol = 1e-4 * np.abs(ref) + 1e-5 + 4 * np.sqrt(kk) * 2.0 ** -24 * terms
        err = np.abs(got.astype(np.float64) - ref)
        assert (err <= tol).all(), f"{what}: max err/tol {np.max(err / tol):.3g}"
    else:
        assert_h16_close(got, ref, what=what)


def _fa_cases(n_cases=10, seed=20261205):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n_cases):
        s = int(rng.choice([1, 17, 64, 100, 191, 256, 300, 513, 777]))
        d = [64, 128][i % 2]
        cases.append((int(rng.integers(1, 3)), int(rng.integers(1, 3)), s, d, bool(i % 3 == 0),
                      "bfloat16" if i % 4 < 2 else "float16"))
    return cases


@pytest.mark.parametrize("b,h,s,d,causal,dtype_name", _fa_cases())
def test_random_attention(device, oracle_mod, b, h, s, d, causal, dtype_name):
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(b * 7 + h * 131 + s * 17 + d)
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal((b, h, s, d), dtype=np.float32), dt) for _ in range(3))
    scale = 1.0 / np.sqrt(d)
    out = torch.full((b, h, s, d), float("nan"), dtype=dt, device=device)
    print(f"[random] attention B={b} H={h} S={s} D={d} causal={causal} {dtype_name}", flush=True)
    native.flash_attention(out, qt.to(device), kt.to(device), vt.to(device), 64, 64, scale, causal)
    ref = oracle_mod.flash_attention_demo(q, k, v, 64, 64, scale=scale, causal=causal)
    got = to_numpy(out)
    assert np.isfinite(got).all()
    assert_within(got, ref, attention_h16_tolerance(q, k, v, scale, causal, dtype_name),
                  what=f"attention {b}x{h}x{s}x{d} causal={causal} {dtype_name}")
