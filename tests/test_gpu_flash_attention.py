"""GPU parity of the gfx950 flash-attention entry (kg_gfx950_flash_attention_entry).

Cases follow the reference's runtime test (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:
571-597: default_rng(2026052901) inputs of shape (1,2,4,3), tiles 2/2), the flash-attention
demos' random shapes (kernel/flash_attention/*.py: S in {257,321,389}, D in {48,64,80}) and
BASELINE configs C4 (bf16 B=4,H=32,S=2048,D=128, non-causal) and C5 (bf16 B=1,H=32,
S=16384, D=128 and 64, causal), all against the oracle's restatement of the demo loop nest
(plus the scale/causal extension), at full size through sampled heads and query blocks.
"""

from __future__ import annotations

import random
from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.golden.make_golden import attention_closed_form
from tests.gpu_util import (assert_f32_close, assert_h16_close, assert_within, attention_f32_tolerance, round_to,
                            to_numpy)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def run(device, dtype, q, k, v, br=64, bc=64, scale=None, causal=False):
    import torch

    qt, kt, vt = (torch.as_tensor(a).to(device) for a in (q, k, v))
    out = torch.full(tuple(qt.shape), float("nan"), dtype=dtype, device=device)
    print(f"[fa] shape={tuple(qt.shape)} {dtype} scale={scale} causal={causal}", flush=True)
    if scale is None and not causal:
        native.call_entry("kg_gfx950_flash_attention_entry", (out, qt, kt, vt, br, bc))
    else:
        native.flash_attention(out, qt, kt, vt, br, bc, 1.0 if scale is None else scale, causal)
    return out


def test_runtime_vector(device):
    import torch

    v = dict(np.load(GOLDEN / "cuda_runtime_vectors.npz"))
    out = run(device, torch.float32, v["fa_q"], v["fa_k"], v["fa_v"], 2, 2)
    # the reference's own bar for this vector (test/cuda/test_cuda_sm89_kernel_demos_runtime.py:595)
    assert_f32_close(to_numpy(out), v["fa_expected"], rtol=1e-4, atol=1e-4, what="runtime vector")
    # the 4-slot form (static demo) gives the same result
    import torch as _t

    qt, kt, vt = (_t.as_tensor(a).to(device) for a in (v["fa_q"], v["fa_k"], v["fa_v"]))
    o4 = _t.empty_like(qt)
    native.call_entry("kg_gfx950_flash_attention_entry", (o4, qt, kt, vt))
    assert_f32_close(to_numpy(o4), v["fa_expected"], rtol=1e-4, atol=1e-4, what="4-slot form")


@pytest.mark.parametrize("seed", [2026052721, 5, 6])
def test_demo_random_profiles_f32(device, oracle_mod, seed):
    """Shapes drawn like kernel/flash_attention/inputs_static_tile_static.py:213-226."""

    import torch

    r = random.Random(seed)
    b, h = r.choice((1, 2)), r.choice((4, 8))
    s, d = r.choice((257, 321, 389)), r.choice((48, 64, 80))
    br, bc = random.Random(seed + 1).choice(((48, 64), (64, 80), (80, 96)))
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((b, h, s, d), dtype=np.float32) for _ in range(3))
    ref = oracle_mod.flash_attention_demo(q, k, v, br, bc)
    tol = attention_f32_tolerance(q, k, v)
    assert_within(to_numpy(run(device, torch.float32, q, k, v, br, bc)), ref, tol, what=str(seed))


@pytest.mark.parametrize("scale,causal", [(0.125, False), (0.3, True), (None, True)])
def test_extensions_f32(device, oracle_mod, scale, causal):
    import torch

    rng = np.random.default_rng(17)
    q, k, v = (rng.standard_normal((1, 3, 200, 40), dtype=np.float32) for _ in range(3))
    ref = oracle_mod.flash_attention_demo(q, k, v, 48, 80, scale=scale, causal=causal)
    out = run(device, torch.float32, q, k, v, 48, 80, scale, causal)
    assert_within(to_numpy(out), ref, attention_f32_tolerance(q, k, v, scale, causal), what=f"scale={scale} causal={causal}")


@pytest.mark.parametrize(
    "shape,s_kv,causal",
    [
        ((1, 2, 256, 128), 256, False),
        ((1, 2, 700, 128), 700, True),  # ragged causal over several 128-query blocks
        ((2, 1, 130, 64), 300, False),  # one partial query block, ragged key tail, S_q != S_kv
        ((1, 1, 1000, 64), 1000, True),
        ((1, 2, 1, 128), 1, False),  # one query, one key
        ((1, 1, 33, 64), 1000, False),
    ],
)
def test_f32_matrix_cores(device, oracle_mod, shape, s_kv, causal):
    """fp32 Q/K/V with D in {64, 128} take the fp32 MFMA kernel; the oracle's demo loop nest
    is the reference where S_q == S_kv, the float64 closed form of the demo's check
    (kernel/flash_attention/inputs_static_tile_static.py:57-87) otherwise."""

    import torch

    b, h, sq, d = shape
    scale = 1.0 / np.sqrt(d)
    rng = np.random.default_rng(sq * 3 + s_kv + d)
    q = rng.standard_normal(shape, dtype=np.float32)
    k, v = (rng.standard_normal((b, h, s_kv, d), dtype=np.float32) for _ in range(2))
    if sq == s_kv:
        ref = oracle_mod.flash_attention_demo(q, k, v, 64, 64, scale=scale, causal=causal)
    else:
        ref = attention_closed_form(q, k, v, scale).astype(np.float32)
    out = run(device, torch.float32, q, k, v, 64, 64, scale, causal)
    assert_within(to_numpy(out), ref, attention_f32_tolerance(q, k, v, scale, causal),
                  what=f"{shape} s_kv={s_kv} causal={causal}")


def test_f32_c4_shape_sampled_heads(device):
    """BASELINE C4's shape (B=4, H=32, S=2048, D=128) in fp32: two heads against the float64
    closed form of the demo's check."""

    import torch

    shape = (4, 32, 2048, 128)
    gen = torch.Generator(device=device).manual_seed(4)
    q, k, v = (torch.randn(shape, generator=gen, device=device) for _ in range(3))
    out = torch.full(shape, float("nan"), device=device)
    print("[fa] f32 C4 shape", flush=True)
    native.flash_attention(out, q, k, v, 64, 64, 1.0 / np.sqrt(128), False)
    for bi, hi in ((0, 0), (3, 31)):
        qh, kh, vh = (to_numpy(t[bi, hi]) for t in (q, k, v))
        ref = attention_closed_form(qh, kh, vh, 1.0 / np.sqrt(128))
        assert_within(to_numpy(out[bi, hi]), ref, attention_f32_tolerance(qh, kh, vh, 1.0 / np.sqrt(128)),
                      what=f"head {bi},{hi}")


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
@pytest.mark.parametrize(
    "shape,causal",
    [
        ((1, 2, 256, 128), False),
        ((1, 2, 512, 128), True),
        ((2, 1, 384, 64), False),
        ((1, 2, 512, 64), True),
        ((1, 1, 300, 128), False),  # ragged S
        ((1, 1, 200, 64), True),  # ragged S, causal
        ((1, 2, 257, 48), False),  # demo-like D
        ((1, 2, 700, 128), True),  # ragged causal over several 256-query blocks
        ((2, 3, 130, 128), False),  # one partial query block, ragged key tail
        ((1, 1, 64, 128), True),  # a single key tile
        ((1, 2, 1, 128), False),  # one query, one key
        ((1, 1, 1000, 64), True),  # D=64 ragged causal over several 128-query blocks
    ],
)
def test_16bit(device, oracle_mod, dtype_name, shape, causal):
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(shape[2] + shape[3])
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), dt) for _ in range(3))
    scale = 1.0 / np.sqrt(shape[3])
    ref = oracle_mod.flash_attention_demo(q, k, v, 64, 64, scale=scale, causal=causal)
    out = run(device, dt, qt, kt, vt, 64, 64, scale, causal)
    assert_h16_close(to_numpy(out), ref, what=f"{dtype_name} {shape} causal={causal}")


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
@pytest.mark.parametrize("shape,causal,scale", [((1, 2, 300, 64), True, 2.0), ((1, 1, 256, 128), False, 0.9),
                                                ((2, 1, 130, 128), True, 0.05)])
def test_16bit_scales(device, oracle_mod, dtype_name, shape, causal, scale):
    """Scales away from 1/sqrt(D) (the kernel scales each fp32 score before its exp2; Q is used
    as stored: multiplying it by the scale in its own 16-bit format would add a rounding of the
    size of the format's unit roundoff to every score, twice the error of the exact scale for
    bf16 on this test's inputs)."""
    import torch

    dt = getattr(torch, dtype_name)
    rng = np.random.default_rng(shape[2] * 7 + shape[3])
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), dt) for _ in range(3))
    ref = oracle_mod.flash_attention_demo(q, k, v, 64, 64, scale=scale, causal=causal)
    out = run(device, dt, qt, kt, vt, 64, 64, scale, causal)
    assert_h16_close(to_numpy(out), ref, what=f"{dtype_name} {shape} causal={causal} scale={scale}")


def _sampled_check(oracle_mod, got, q, k, v, heads, blocks, scale, causal, name):
    for (b, h) in heads:
        for m0, m1 in blocks:
            ref = oracle_mod.flash_attention_demo(
                q[b : b + 1, h : h + 1], k[b : b + 1, h : h + 1], v[b : b + 1, h : h + 1], 64, 64,
                scale=scale, causal=causal, threads=1, m_range=(m0, m1),
            )
            assert_h16_close(got[b, h, m0:m1], ref[0, 0, m0:m1], what=f"{name} b={b} h={h} rows {m0}:{m1}")


def test_c4_full_size(device, oracle_mod):
    import torch

    shape = (4, 32, 2048, 128)
    rng = np.random.default_rng(20261205)
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), torch.bfloat16) for _ in range(3))
    scale = 1.0 / np.sqrt(128.0)
    got = to_numpy(run(device, torch.bfloat16, qt, kt, vt, 128, 64, scale, False))
    assert np.isfinite(got).all()
    _sampled_check(oracle_mod, got, q, k, v, [(0, 0), (3, 31)], [(0, 64), (1984, 2048)], scale, False, "C4")
    # every output row is a convex combination of V rows: it lies inside V's per-column range
    vmin = v.min(axis=2, keepdims=True)
    vmax = v.max(axis=2, keepdims=True)
    slack = 1e-2 * (vmax - vmin)
    assert ((got >= vmin - slack) & (got <= vmax + slack)).all()


@pytest.mark.parametrize(
    "shape,causal",
    [((2, 64, 1000, 128), False), ((1, 128, 700, 128), True), ((1, 8, 2048, 128), False)],
    ids=["8wave_ragged", "8wave_ragged_causal", "4wave_small_grid"],
)
def test_workgroup_shapes_d128(device, oracle_mod, shape, causal):
    """D=128 takes 8-wave workgroups (256 queries) when they give every CU one and 4-wave
    workgroups (128 queries) otherwise: the first two shapes are 512 and 384 ragged 8-wave
    workgroups, the third 128 4-wave ones. Sampled heads and row blocks against the oracle."""

    import torch

    b, h, s, d = shape
    rng = np.random.default_rng(s + h)
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), torch.bfloat16) for _ in range(3))
    scale = 1.0 / np.sqrt(128.0)
    got = to_numpy(run(device, torch.bfloat16, qt, kt, vt, 128, 64, scale, causal))
    assert np.isfinite(got).all()
    heads = [(0, 0), (b - 1, h - 1)]
    blocks = [(0, 64), (s - 64 - s % 7, s - s % 7), (s - 40, s)]
    _sampled_check(oracle_mod, got, q, k, v, heads, blocks, scale, causal, f"{shape}")


@pytest.mark.parametrize("d,seed", [(128, 20261206), (64, 20261207)])
def test_c5_full_size_causal(device, oracle_mod, d, seed):
    import torch

    shape = (1, 32, 16384, d)
    rng = np.random.default_rng(seed)
    (qt, q), (kt, k), (vt, v) = (round_to(rng.standard_normal(shape, dtype=np.float32), torch.bfloat16) for _ in range(3))
    scale = 1.0 / np.sqrt(float(d))
    got = to_numpy(run(device, torch.bfloat16, qt, kt, vt, 128, 64, scale, True))
    assert np.isfinite(got).all()
    _sampled_check(oracle_mod, got, q, k, v, [(0, 0), (0, 21)], [(0, 64), (8192, 8256), (16320, 16384)], scale, True,
                   f"C5 D={d}")
    # causal row 0 attends only to key 0: out[:, :, 0] == V[:, :, 0] (bf16-rounded)
    np.testing.assert_allclose(got[0, :, 0, :], v[0, :, 0, :], rtol=1e-2, atol=1e-2)


PERSISTENT = [
    ((1, 65, 2048, 128), 2048, "bfloat16"),  # 520 items on 256 workgroups: 8 of them take a third
    ((2, 64, 2048, 128), 2048, "float16"),   # 1024 items, 4 per workgroup
    ((1, 64, 2048, 128), 256, "bfloat16"),   # 4 key tiles per item, the fewest: Q staged in tiles 0-1
    ((1, 64, 2048, 128), 384, "float16"),    # 6 key tiles per item
    ((1, 64, 2048, 128), 128, "bfloat16"),   # 2 key tiles: too few, one workgroup per item
    ((1, 130, 1024, 64), 1024, "bfloat16"),  # D=64: 1040 items on 512 four-wave workgroups
]


@pytest.mark.parametrize("shape,s_kv,dtype", PERSISTENT)
def test_persistent_form_matches_one_item_per_workgroup(device, oracle_mod, shape, s_kv, dtype):
    """Non-causal whole-tile attention with an even key-tile count of at least 4 and at least
    two items (query blocks) per workgroup slot runs persistent workgroups: each walks the
    items gridDim.x apart as one sequence of key tiles (the next item's Q staged in LDS during
    tiles nt-4 and nt-3, its K tiles 0-1 and V tile 0 copied and its first S tile computed in
    this item's last two tiles). A three-deep ring (memory_stage=3) launches one workgroup per
    item instead.
    Both do the same arithmetic per item, so the bits must agree; sampled rows of two heads
    also against the oracle (S_kv = S_q: the demo's loop nest) or the float64 formula."""

    import torch

    tdt = getattr(torch, dtype)
    b, h, s, d = shape
    rng = np.random.default_rng(s + h + s_kv)
    q, qn = round_to(rng.standard_normal(shape, dtype=np.float32), tdt)
    (k, kn), (v, vn) = (round_to(rng.standard_normal((b, h, s_kv, d), dtype=np.float32), tdt) for _ in range(2))
    q, k, v = (t.to(device) for t in (q, k, v))
    scale = 1.0 / np.sqrt(d)
    outs = []
    for stages in (2, 3):
        out = torch.full(shape, float("nan"), dtype=tdt, device=device)
        print(f"[fa] persistent check {shape} s_kv={s_kv} {dtype} memory_stage={stages}", flush=True)
        native.flash_attention(out, q, k, v, 64, 64, scale, False, memory_stage=stages)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    got = to_numpy(outs[0])
    assert np.isfinite(got).all()
    heads, blocks = [(0, 0), (b - 1, h - 1)], [(0, 64), (s - 64, s)]
    if s_kv == s:
        _sampled_check(oracle_mod, got, qn, kn, vn, heads, blocks, scale, False, f"{shape}")
        return
    for bb, hh in heads:
        for m0, m1 in blocks:
            logits = qn[bb, hh, m0:m1].astype(np.float64) @ kn[bb, hh].astype(np.float64).T * scale
            w = np.exp(logits - logits.max(axis=1, keepdims=True))
            ref = (w / w.sum(axis=1, keepdims=True)) @ vn[bb, hh].astype(np.float64)
            assert_h16_close(got[bb, hh, m0:m1], ref, what=f"{shape} s_kv={s_kv} b={bb} h={hh} rows {m0}:{m1}")


def test_rejects_bad_args(device):
    import torch

    q = torch.zeros(1, 1, 8, 4, device=device)
    o = torch.zeros(1, 1, 8, 4, device=device)
    with pytest.raises(native.NativeLibraryError):
        native.flash_attention(o, q, q, q, 0, 4)
    with pytest.raises(native.NativeLibraryError):
        native.call_entry("kg_gfx950_flash_attention_entry", (o, q, q, q, 4, 4, 1.0, 2))
