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
