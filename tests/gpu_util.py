"""Helpers shared by the GPU parity tests (no GPU work at import time)."""

from __future__ import annotations

import numpy as np

# Tolerances:
#   fp32 kernels: |out - oracle| <= 1e-5 + 1e-4 * |oracle|
#   bf16/fp16 kernels: |out - oracle| <= 2e-2 * |oracle| + 1e-2 * rms(oracle), where the
#   oracle computes in fp32 on the identically rounded 16-bit inputs. The rms term bounds
#   the absolute error of elements that cancel to ~0 (fp32 summation order, 16-bit P in
#   attention); it is 1% of the typical output magnitude.
F32_RTOL, F32_ATOL = 1e-4, 1e-5
H16_RTOL, H16_ATOL_RMS = 2e-2, 1e-2


def to_numpy(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_f32_close(out, ref, rtol: float = F32_RTOL, atol: float = F32_ATOL, what: str = "") -> None:
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    err = np.abs(out - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; max err {err.max():.3e}"


def assert_h16_close(out, ref, what: str = "") -> None:
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    atol = H16_ATOL_RMS * rms
    err = np.abs(out - ref)
    bad = err > atol + H16_RTOL * np.abs(ref)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside rtol={H16_RTOL} atol={atol:.3e}; max err {err.max():.3e}"
    )


def round_to(x: np.ndarray, torch_dtype):
    """Round fp32 data to a 16-bit torch dtype (RNE) and return (tensor16_cpu, exact fp32 copy)."""

    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch_dtype)
    return t, t.float().numpy()


def attention_f32_tolerance(q, k, v, scale=None, causal=False) -> np.ndarray:
    """Per-element fp32 attention bar for kernels whose sums run in another order than the
    oracle's sequential loops (MFMA dot products, exp2, tiled online softmax).

    |out - oracle| <= 1e-5 + 1e-4 |oracle| (the north-star fp32 bar) plus first-order
    rounding terms, all from float64 quantities of the inputs (Higham & Mary's probabilistic
    bound 4 sqrt(n) 2^-24 for an n-term fp32 sum in any order):
      - a score s_ij = scale * sum_d q_id k_jd off by e_ij moves O_i by at most
        max_j e_ij * (P |V - O|)_i, with e_ij = 4 sqrt(D) 2^-24 scale (|Q| |K|^T)_ij plus
        the exp argument's rounding, |s_ij - m_i| * log2(e) * 2^-24 + 2^-22 (exp2 and its
        result each within an ulp);
      - the P V sum over S_kv keys in any order: 4 sqrt(S_kv) 2^-24 (P |V|)_i / 1.
    q, k, v: float arrays [..., S, D]; returns the atol array for the output shape."""

    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s_q, d = q.shape[-2], q.shape[-1]
    s_kv = k.shape[-2]
    sc = 1.0 if scale is None else float(scale)
    s = sc * (q @ np.swapaxes(k, -1, -2))
    if causal:
        mask = np.tril(np.ones((s_q, s_kv), bool))
        s = np.where(mask, s, -np.inf)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    p /= p.sum(-1, keepdims=True)
    o = p @ v
    dots = sc * (np.abs(q) @ np.swapaxes(np.abs(k), -1, -2))
    arg = np.where(np.isfinite(s), np.abs(s - m), 0.0) * 1.4426950408889634
    e = 4 * np.sqrt(d) * 2.0 ** -24 * dots + arg * 2.0 ** -24 + 2.0 ** -22
    if causal:
        e = np.where(mask, e, 0.0)
    e_max = e.max(-1, keepdims=True)
    dev = p @ np.abs(v) + np.abs(o)  # bounds (P |V - O|)_i elementwise
    return 1e-5 + 1e-4 * np.abs(o) + e_max * dev + 4 * np.sqrt(s_kv) * 2.0 ** -24 * (p @ np.abs(v))


def attention_h16_tolerance(q, k, v, scale=None, causal=False, dtype_name="bfloat16") -> np.ndarray:
    """Per-element bar for the 16-bit attention kernels: the north-star 2e-2 |oracle| +
    1e-2 rms(oracle), plus the first-order effect of the one rounding the design adds on top
    of the output's own: P is rounded to the 16-bit format (P_j (1 + d_j), |d_j| <= u, the
    unit roundoff of round-to-nearest: 2^-8 for bf16's 8-bit significand, 2^-11 for f16's 11
    bits) before the P V product, and the row sum uses the same rounded P, so
    O_i = sum_j w~_j V_j moves by sum_j w_j d_j (V_j - O_i) to first order. The d_j are
    rounding errors of different values, taken as independent with mean 0 (|d_j| <= u,
    variance at most u^2 / 3): the probabilistic bound with the usual factor of 4 standard
    deviations is 4 u sqrt(sum_j w_j^2 (V_j - O_i)^2). That term covers short causal rows
    (row i averages i + 1 keys with large weights, where the rms term alone is too tight)
    and shrinks on long rows like 1 / sqrt(keys). Float64 from the inputs."""

    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s_q, s_kv = q.shape[-2], k.shape[-2]
    sc = 1.0 if scale is None else float(scale)
    s = sc * (q @ np.swapaxes(k, -1, -2))
    if causal:
        s = np.where(np.tril(np.ones((s_q, s_kv), bool)), s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    o = w @ v
    rms = float(np.sqrt(np.mean(o * o))) if o.size else 0.0
    u = {"bfloat16": 2.0 ** -8, "float16": 2.0 ** -11}[dtype_name]
    w2 = w * w
    # sum_j w_j^2 (V_j - O)^2 = W2 V^2 - 2 O (W2 V) + O^2 (W2 1), clipped at 0 against cancellation
    spread = np.maximum(w2 @ (v * v) - 2 * o * (w2 @ v) + o * o * w2.sum(-1, keepdims=True), 0.0)
    return H16_ATOL_RMS * rms + H16_RTOL * np.abs(o) + 4 * u * np.sqrt(spread)


def assert_within(out, ref, atol, what: str = "") -> None:
    """|out - ref| <= atol elementwise (atol an array from a documented error bound)."""

    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    err = np.abs(out - ref)
    bad = ~(err <= atol)
    if bad.any():
        worst = np.unravel_index(np.argmax(np.where(bad, err / np.maximum(atol, 1e-30), 0)), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside the bound; worst err {err[worst]:.3e} "
                             f"> {np.broadcast_to(atol, err.shape)[worst]:.3e} at {worst}")
