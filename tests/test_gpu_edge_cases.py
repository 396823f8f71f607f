"""GPU edge cases of the three entries beyond the reference's demo shapes: strided and
transposed operands (the memory-slot contract carries element strides,
kernel_gen/execute_engine/runtime_args.py:395-430), degenerate extents (K = 0, M = 0,
empty attention), and attention with different query and key lengths (an extension:
the reference's demos use one S). Expected values come from the oracle on contiguous
copies or, where the oracle's demo loop nest has no such case, from the float64 closed
form of the demo's reference check (kernel/flash_attention/inputs_static_tile_static.py:
57-87)."""

from __future__ import annotations

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.golden.make_golden import attention_closed_form
from tests.gpu_util import assert_f32_close, assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype_name,rhs_layout", [("float32", "transposed"), ("bfloat16", "transposed"),
                                                   ("bfloat16", "contiguous")])
def test_matmul_strided_and_transposed_operands(device, oracle_mod, dtype_name, rhs_layout):
    """lhs is a column window of a wider matrix (row stride 112, 16-byte offset); rhs is a
    transposed view (element strides (1, K): the generic kernel) or contiguous (the MFMA
    kernel with a leading dimension other than K)."""

    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(41)
    m, k, n = 150, 72, 96
    a_wide = rng.standard_normal((m, k + 40)).astype(np.float32)  # lhs = a_wide[:, 8:8+k], row stride k+40
    bt = rng.standard_normal((n, k)).astype(np.float32)  # rhs = bt^T
    at_dev, a_wide = round_to(a_wide, dt) if dt != torch.float32 else (torch.from_numpy(a_wide), a_wide)
    bt_dev, bt = round_to(bt, dt) if dt != torch.float32 else (torch.from_numpy(bt), bt)
    lhs = at_dev.to(device)[:, 8:8 + k]
    rhs = bt_dev.to(device).t()
    if rhs_layout == "contiguous":
        rhs = rhs.contiguous()
    assert not lhs.is_contiguous() and rhs.is_contiguous() == (rhs_layout == "contiguous")
    out = torch.full((m, n), float("nan"), dtype=dt, device=device)
    print(f"[edge] matmul strided {dtype_name} lhs.stride={lhs.stride()} rhs.stride={rhs.stride()}", flush=True)
    native.matmul(out, lhs, rhs, None)
    ref = oracle_mod.matmul_demo(np.ascontiguousarray(a_wide[:, 8:8 + k]), np.ascontiguousarray(bt.T), None, (64, 64, 64))
    if dt == torch.float32:
        assert_f32_close(to_numpy(out), ref, rtol=1e-4, atol=1e-5, what="strided f32")
    else:
        assert_h16_close(to_numpy(out), ref, what="strided bf16")


def test_matmul_degenerate_extents(device):
    import torch

    bias = torch.arange(8, dtype=torch.float32, device=device)
    lhs = torch.empty(5, 0, device=device)
    rhs = torch.empty(0, 8, device=device)
    out = torch.full((5, 8), float("nan"), device=device)
    print("[edge] matmul K=0 with bias", flush=True)
    native.matmul(out, lhs, rhs, bias)  # empty sum: out = bias in every row
    assert torch.equal(out, bias.expand(5, 8))
    out0 = torch.empty(0, 8, device=device)
    print("[edge] matmul M=0", flush=True)
    native.matmul(out0, torch.empty(0, 3, device=device), torch.ones(3, 8, device=device), None)


@pytest.mark.parametrize(
    "dtype_name,b,h,sq,skv,d",
    [("bfloat16", 1, 2, 100, 300, 64), ("bfloat16", 2, 1, 260, 70, 128), ("float16", 1, 1, 33, 1000, 128),
     ("float32", 1, 3, 50, 77, 40)],
)
def test_attention_different_query_and_key_lengths(device, dtype_name, b, h, sq, skv, d):
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(sq * 7 + skv)
    scale = 1.0 / np.sqrt(d)
    arrays = [rng.standard_normal(s, dtype=np.float32) for s in ((b, h, sq, d), (b, h, skv, d), (b, h, skv, d))]
    if dt == torch.float32:
        tq, tk, tv = (torch.from_numpy(a) for a in arrays)
        q, k, v = arrays
    else:
        (tq, q), (tk, k), (tv, v) = (round_to(a, dt) for a in arrays)
    out = torch.full((b, h, sq, d), float("nan"), dtype=dt, device=device)
    print(f"[edge] attention {dtype_name} q={tuple(tq.shape)} kv={tuple(tk.shape)}", flush=True)
    native.flash_attention(out, tq.to(device), tk.to(device), tv.to(device), 64, 64, scale, False)
    ref = attention_closed_form(q, k, v, scale)
    if dt == torch.float32:
        assert_f32_close(to_numpy(out), ref.astype(np.float32), rtol=1e-4, atol=1e-4, what="f32 sq!=skv")
    else:
        assert_h16_close(to_numpy(out), ref.astype(np.float32), what=f"{dtype_name} sq!=skv")


def test_attention_empty_and_causal_length_mismatch(device):
    import torch

    q = torch.empty(1, 2, 0, 64, dtype=torch.bfloat16, device=device)
    print("[edge] attention S=0", flush=True)
    native.flash_attention(torch.empty_like(q), q, q, q, 64, 64, 0.125, False)
    q1 = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device=device)
    kv = torch.zeros(1, 1, 9, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(native.NativeLibraryError, match="causal"):
        native.flash_attention(torch.empty_like(q1), q1, kv, kv, 64, 64, 0.125, True)
    no_keys = torch.empty(1, 1, 0, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(native.NativeLibraryError, match="no keys"):
        native.flash_attention(torch.empty_like(q1), q1, no_keys, no_keys, 64, 64, 0.125, False)
