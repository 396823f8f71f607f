"""GPU parity of the gfx950 matmul entry (kg_gfx950_matmul_entry) against the CPU oracle.

Slot order and cases follow the reference's runtime test
(test/cuda/test_cuda_sm89_kernel_demos_runtime.py:499-527) and the matmul demos
(kernel/matmul/*.py); BASELINE configs C1 (fp32 256^3), C2 (bf16 4096^3) and C2' (bf16
8192x1024x4096) are checked at full size through sampled output tiles against the oracle
and through size-independent properties.
"""

from __future__ import annotations

import random
from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd import native
from tests.gpu_util import assert_f32_close, assert_h16_close, round_to, to_numpy

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def run(device, out_dtype, lhs, rhs, bias=None, tiles=()):
    import torch

    lt = torch.as_tensor(lhs).to(device)
    rt = torch.as_tensor(rhs).to(device)
    bt = None if bias is None else torch.as_tensor(bias).to(device)
    out = torch.full((lt.shape[0], rt.shape[1]), float("nan"), dtype=out_dtype, device=device)
    print(f"[matmul] M={lt.shape[0]} K={lt.shape[1]} N={rt.shape[1]} {out_dtype} bias={bias is not None}", flush=True)
    native.matmul(out, lt, rt, bt, *tiles)
    return out


def test_runtime_vectors(device, oracle_mod):
    import torch

    v = dict(np.load(GOLDEN / "cuda_runtime_vectors.npz"))
    for bias, key in ((None, "matmul_absent"), (v["matmul_bias"], "matmul_present")):
        out = run(device, torch.float32, v["matmul_lhs"], v["matmul_rhs"], bias, (2, 2, 2))
        assert_f32_close(to_numpy(out), v[key], rtol=1e-5, atol=1e-5, what=key)


def test_demo_static_shape_f32(device, oracle_mod):
    import torch

    rng = np.random.default_rng(2026051601)
    lhs = rng.normal(size=(166, 217)).astype(np.float32)
    rhs = rng.normal(size=(217, 172)).astype(np.float32)
    bias = rng.normal(size=(172,)).astype(np.float32)
    for b in (None, bias):
        ref = oracle_mod.matmul_demo(lhs, rhs, b, (48, 80, 56))
        out = run(device, torch.float32, lhs, rhs, b, (48, 80, 56))
        assert_f32_close(to_numpy(out), ref, what="demo 166x217x172")


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_dynamic_shapes_f32(device, oracle_mod, seed):
    import torch

    r = random.Random(seed)
    m, k, n = r.randint(160, 256), r.randint(160, 256), r.randint(160, 256)
    tiles = r.choice(((72, 56, 48), (48, 80, 56)))
    rng = np.random.default_rng(seed)
    lhs = rng.normal(size=(m, k)).astype(np.float32)
    rhs = rng.normal(size=(k, n)).astype(np.float32)
    bias = rng.normal(size=(n,)).astype(np.float32)
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, tiles)
    assert_f32_close(to_numpy(run(device, torch.float32, lhs, rhs, bias, tiles)), ref, what=f"{m}x{k}x{n}")


def test_c1_fp32_256(device, oracle_mod):
    import torch

    rng = np.random.default_rng(20261201)
    a = rng.uniform(-1, 1, size=(256, 256)).astype(np.float32)
    b = rng.uniform(-1, 1, size=(256, 256)).astype(np.float32)
    ref = oracle_mod.matmul_demo(a, b, None, (64, 64, 64))
    assert_f32_close(to_numpy(run(device, torch.float32, a, b)), ref, what="C1")


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
@pytest.mark.parametrize(
    "shape",
    [(2, 3, 4), (1, 8, 8), (300, 136, 264), (256, 64, 256), (512, 128, 512), (257, 72, 8), (64, 520, 1032)],
)
@pytest.mark.parametrize("bias_kind", ["none", "f32", "same"])
def test_16bit_shapes(device, oracle_mod, dtype_name, shape, bias_kind):
    import torch

    dt = getattr(torch, dtype_name)
    m, k, n = shape
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    lt, lhs = round_to(rng.normal(size=(m, k)) * 0.5, dt)
    rt, rhs = round_to(rng.normal(size=(k, n)) * 0.5, dt)
    bias = None
    bt = None
    if bias_kind == "f32":
        bias = rng.normal(size=(n,)).astype(np.float32)
        bt = bias
    elif bias_kind == "same":
        bt16, bias = round_to(rng.normal(size=(n,)), dt)
        bt = bt16
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, (64, 64, 64))
    out = run(device, dt, lt, rt, bt)
    assert_h16_close(to_numpy(out), ref, what=f"{dtype_name} {shape} bias={bias_kind}")


@pytest.mark.parametrize("bias_kind", ["f32", "same"])
def test_pipe_256_row_tiles_with_bias(device, oracle_mod, bias_kind):
    """4096 x 4096 outputs are 256 tiles of 256 x 256 (one per CU): the 256-row pipelined
    path; smaller aligned shapes above take its 128-row tiles."""

    import torch

    m, k, n = 4096, 64, 4096
    rng = np.random.default_rng(91)
    lt, lhs = round_to(rng.normal(size=(m, k)) * 0.5, torch.bfloat16)
    rt, rhs = round_to(rng.normal(size=(k, n)) * 0.5, torch.bfloat16)
    if bias_kind == "f32":
        bias = rng.normal(size=(n,)).astype(np.float32)
        bt = bias
    else:
        bt, bias = round_to(rng.normal(size=(n,)), torch.bfloat16)
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, (64, 64, 64))
    out = run(device, torch.bfloat16, lt, rt, bt)
    assert_h16_close(to_numpy(out), ref, what=f"4096x64x4096 bias={bias_kind}")


@pytest.mark.parametrize(
    "dtype_name,bias_kind,k",
    [("bfloat16", None, 1024), ("float16", "same", 1024), ("bfloat16", "f32", 1024), ("bfloat16", None, 256),
     ("float16", None, 1056)],
    ids=["bf16-k1024", "f16-bias16-k1024", "bf16-bias32-k1024", "bf16-k256", "f16-k1056"])
def test_four_wave_tiles_match_eight_wave_kernel(device, dtype_name, bias_kind, k):
    """Whole 256 x 256 tiles that fill the chip run on four waves of 128 x 128; the same rows
    computed as a 1024-row matmul of their own (64 tiles of 256 x 256, too few for the chip:
    the eight-wave kernel's 128-row tiles, K not split) must give the same bits: both issue
    one 16x16x32 MFMA per 32-deep slice and output block, in k order, and round once.
    K = 1024 and 256 (32 and 8 slices: the exact-K form, whose last four slices are one
    compile-time group; 8 is the fewest it takes) and 1056 (33 slices: the general loop)."""

    import torch

    tdt = getattr(torch, dtype_name)
    m, n = 4096, 4096
    g = torch.Generator(device=device).manual_seed(77)
    a = (torch.randn(m, k, generator=g, device=device) * 0.1).to(tdt)
    b = (torch.randn(k, n, generator=g, device=device) * 0.1).to(tdt)
    bias = None
    if bias_kind == "f32":
        bias = torch.randn(n, generator=g, device=device)
    elif bias_kind == "same":
        bias = torch.randn(n, generator=g, device=device).to(tdt)
    full = torch.full((m, n), float("nan"), dtype=tdt, device=device)
    native.matmul(full, a, b, bias)
    for r0 in (0, 3072):
        part = torch.full((1024, n), float("nan"), dtype=tdt, device=device)
        print(f"[matmul] four-wave vs eight-wave rows {r0}:{r0 + 1024} {dtype_name} bias={bias_kind} k={k}", flush=True)
        native.matmul(part, a[r0:r0 + 1024].contiguous(), b, bias)
        assert torch.equal(full[r0:r0 + 1024], part), f"rows {r0}:{r0 + 1024}"


@pytest.mark.parametrize(
    "dtype_name,bias_kind,k",
    [("bfloat16", None, 1024), ("float16", "f32", 1024), ("bfloat16", "same", 1056)],
    ids=["bf16-k1024", "f16-bias32-k1024", "bf16-bias16-k1056"])
def test_four_wave_128_row_tiles_match_eight_wave_kernel(device, dtype_name, bias_kind, k):
    """Outputs whose 256 x 256 tiles would leave CUs idle but whose 128 x 256 tiles fill the
    chip (2048 x 4096: 128 and 256 tiles) run on four waves of 64 x 128; the same rows
    computed again as a ragged 1000-row matmul (the eight-wave kernel's ragged form, 128
    tiles, K not split) must give the same bits: both issue one 16x16x32 MFMA per 32-deep
    slice and output block, in k order, and round once. K = 1024 is the exact-K form, 1056
    the general loop."""

    import torch

    tdt = getattr(torch, dtype_name)
    m, n = 2048, 4096
    g = torch.Generator(device=device).manual_seed(78)
    a = (torch.randn(m, k, generator=g, device=device) * 0.1).to(tdt)
    b = (torch.randn(k, n, generator=g, device=device) * 0.1).to(tdt)
    bias = None
    if bias_kind == "f32":
        bias = torch.randn(n, generator=g, device=device)
    elif bias_kind == "same":
        bias = torch.randn(n, generator=g, device=device).to(tdt)
    full = torch.full((m, n), float("nan"), dtype=tdt, device=device)
    print(f"[matmul] four-wave 128-row tiles {m}x{n}x{k} {dtype_name} bias={bias_kind}", flush=True)
    native.matmul(full, a, b, bias)
    for r0 in (0, 1048):
        part = torch.full((1000, n), float("nan"), dtype=tdt, device=device)
        print(f"[matmul] eight-wave ragged rows {r0}:{r0 + 1000}", flush=True)
        native.matmul(part, a[r0:r0 + 1000].contiguous(), b, bias)
        assert torch.equal(full[r0:r0 + 1000], part), f"rows {r0}:{r0 + 1000}"


@pytest.mark.parametrize(
    "shape,dtype_name,bias_kind,rows",
    [
        ((16, 4096, 4096), "bfloat16", "f32", None),  # 16 tiles: 16 K chunks of 256
        ((128, 8192, 1024), "float16", "same", [(0, 16), (112, 128)]),  # 4 tiles: 32 chunks
        ((3, 1000, 136), "bfloat16", "none", None),  # one ragged tile, last chunk 8 deep short of a slice
        ((40, 2048, 520), "float16", "f32", None),  # 3 tiles, ragged N
        ((2048, 4096, 2048), "bfloat16", "f32", [(0, 16), (2032, 2048)]),  # 128 tiles, long K: 2 chunks
    ],
    ids=["16x4096x4096", "128x8192x1024", "3x1000x136", "40x2048x520", "2048x4096x2048"],
)
def test_split_k_skinny(device, oracle_mod, shape, dtype_name, bias_kind, rows):
    """Outputs of few tiles run the pipelined kernel split over K (fp32 partial sums in a
    stream-ordered workspace, added in chunk order by a second kernel that also adds the bias
    and rounds once). The output is a window of a NaN-filled buffer (extra rows and columns
    must stay NaN); rows are checked against the oracle."""

    import torch

    dt = getattr(torch, dtype_name)
    m, k, n = shape
    rng = np.random.default_rng(m + 5 * k + 11 * n)
    lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.1, dt)
    rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.1, dt)
    bias = bt = None
    if bias_kind == "f32":
        bias = bt = rng.standard_normal(n).astype(np.float32)
    elif bias_kind == "same":
        bt, bias = round_to(rng.standard_normal(n), dt)
    big = torch.full((m + 2, n + 8), float("nan"), dtype=dt, device=device)
    out = big[:m, :n]
    print(f"[matmul] split-K M={m} K={k} N={n} {dtype_name} bias={bias_kind}", flush=True)
    native.matmul(out, lt.to(device), rt.to(device), None if bt is None else torch.as_tensor(bt).to(device))
    got = to_numpy(big)
    assert np.isnan(got[m:]).all() and np.isnan(got[:, n:]).all(), "store outside the output window"
    for r0, r1 in rows or [(0, m)]:
        ref = oracle_mod.matmul_demo(lhs[r0:r1], rhs, bias, (64, 64, 64))
        assert_h16_close(got[r0:r1, :n], ref, what=f"{shape} rows {r0}:{r1}")
    # the same call again gives the same bits (chunks are added in a fixed order)
    again = torch.full_like(out, float("nan"))
    native.matmul(again, lt.to(device), rt.to(device), None if bt is None else torch.as_tensor(bt).to(device))
    assert torch.equal(again, out.contiguous())


def test_split_k_on_many_streams(device, oracle_mod):
    """Split-K matmuls enqueued on more streams than the library keeps workspaces for (8 per
    device): the ninth and later streams take over the least recently used workspace, whose
    buffer is released only after the device's pending work. Two rounds over 11 streams, each
    call with its own inputs, every output checked against the oracle."""

    import torch

    m, k, n = 16, 2048, 512  # 2 output tiles, K split 8 ways
    streams = [torch.cuda.Stream(device=device) for _ in range(11)]
    cases = []
    for rnd in range(2):
        for i, stream in enumerate(streams):
            rng = np.random.default_rng(1000 * rnd + i)
            lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.1, torch.bfloat16)
            rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.1, torch.bfloat16)
            a, b = lt.to(device), rt.to(device)
            out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
            torch.cuda.synchronize()
            print(f"[matmul] split-K round {rnd} stream {i}", flush=True)
            native.set_launch_mode(False, stream.cuda_stream)
            try:
                native.matmul(out, a, b, None)
            finally:
                native.set_launch_mode(True, None)
            cases.append((out, lhs, rhs, (rnd, i), (a, b)))  # inputs stay alive until the sync
    torch.cuda.synchronize()
    for out, lhs, rhs, tag, _ in cases:
        ref = oracle_mod.matmul_demo(lhs, rhs, None, (64, 64, 64))
        assert_h16_close(to_numpy(out), ref, what=f"split-K round/stream {tag}")


@pytest.mark.parametrize(
    "shape,rows",
    [
        ((1000, 520, 1000), None),  # 128-row tiles, every edge ragged, 8-deep last K slice
        ((4224, 40, 4104), None),  # 256-row tiles, half a last tile row, 8 columns over, K = 40
        ((520, 4096, 776), None),  # 128-row tiles, long K
        ((4000, 4000, 4000), [(0, 32), (3968, 4000)]),  # 256-row tiles, ragged M and N
    ],
    ids=["1000x520x1000", "4224x40x4104", "520x4096x776", "4000^3"],
)
def test_ragged_edges_store_only_inside(device, oracle_mod, shape, rows):
    """Shapes that are not tile multiples take the pipelined kernel's ragged mode: edge copies
    land zeros and the epilogue masks its stores. The output is a window of a NaN-filled
    buffer with 3 extra rows and 8 extra columns, which must stay NaN."""

    import torch

    m, k, n = shape
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.1, torch.bfloat16)
    rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.1, torch.bfloat16)
    bias = rng.standard_normal(n).astype(np.float32)
    big = torch.full((m + 3, n + 8), float("nan"), dtype=torch.bfloat16, device=device)
    out = big[:m, :n]
    print(f"[matmul] ragged M={m} K={k} N={n} ldc={n + 8}", flush=True)
    native.matmul(out, lt.to(device), rt.to(device), torch.from_numpy(bias).to(device))
    got = to_numpy(big)
    assert np.isnan(got[m:]).all() and np.isnan(got[:, n:]).all(), "store outside the output window"
    for r0, r1 in rows or [(0, m)]:
        ref = oracle_mod.matmul_demo(lhs[r0:r1], rhs, bias, (64, 64, 64))
        assert_h16_close(got[r0:r1, :n], ref, what=f"{shape} rows {r0}:{r1}")


@pytest.mark.parametrize(
    "shape,rows,with_bias",
    [
        ((1024, 256, 1024), None, False),  # 64 aligned 128 x 128 tiles
        ((1000, 520, 1000), None, True),  # every edge ragged, 8-deep last K slice
        ((777, 64, 2052), None, True),  # 4 columns past the last full tile
        ((4096, 4096, 4096), [(0, 32), (4064, 4096)], False),
        ((1024, 300, 1000), None, True),  # lhs and rhs as column windows of wider buffers
    ],
    ids=["1024x256x1024", "1000x520x1000", "777x64x2052", "4096^3", "strided"],
)
def test_f32_matrix_core_shapes(device, oracle_mod, shape, rows, with_bias):
    """fp32 operands large enough for the fp32 MFMA kernel (v_mfma_f32_32x32x2_f32), which
    sums K in a different order than the oracle's sequential loop. Tolerance: the demo's
    rtol 1e-4 / atol 1e-5 plus the rounding that two fp32 summation orders of K products can
    differ by, 4 sqrt(K) 2^-24 (|A| |B|)[m, n] (the probabilistic bound of Higham and Mary,
    SIAM J. Sci. Comput. 41 (2019)): it reaches 1e-4 of the result only where K is large and
    the result is small against its terms. The output is a window of a NaN-filled buffer
    (3 extra rows, 4 extra columns) that must stay NaN outside it."""

    import torch

    m, k, n = shape
    rng = np.random.default_rng(m + 5 * k + 11 * n)
    lhs = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    rhs = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32) if with_bias else None
    big = torch.full((m + 3, n + 4), float("nan"), dtype=torch.float32, device=device)
    out = big[:m, :n]
    lt, rt = torch.from_numpy(lhs).to(device), torch.from_numpy(rhs).to(device)
    if shape == (1024, 300, 1000):  # the "strided" case: row strides k + 12 and n + 20 (multiples of 4)
        lt = torch.cat([lt, torch.zeros(m, 12, device=device)], 1)[:, :k]
        rt = torch.cat([rt, torch.zeros(k, 20, device=device)], 1)[:, :n]
        assert not lt.is_contiguous() and not rt.is_contiguous()
    print(f"[matmul] f32 matrix cores M={m} K={k} N={n} bias={with_bias} lda={lt.stride(0)} ldb={rt.stride(0)}", flush=True)
    native.matmul(out, lt, rt, None if bias is None else torch.from_numpy(bias).to(device))
    got = to_numpy(big)
    assert np.isnan(got[m:]).all() and np.isnan(got[:, n:]).all(), "store outside the output window"
    for r0, r1 in rows or [(0, m)]:
        ref = oracle_mod.matmul_demo(np.ascontiguousarray(lhs[r0:r1]), rhs, bias, (64, 64, 64))
        terms = np.abs(lhs[r0:r1]).astype(np.float64) @ np.abs(rhs).astype(np.float64)
        tol = 1e-4 * np.abs(ref) + 1e-5 + 4 * np.sqrt(k) * 2.0 ** -24 * terms
        err = np.abs(got[r0:r1, :n].astype(np.float64) - ref)
        worst = np.unravel_index(np.argmax(err - tol), err.shape)
        assert (err <= tol).all(), f"{shape} rows {r0}:{r1}: err {err[worst]:.3g} > tol {tol[worst]:.3g} at {worst}"


@pytest.mark.parametrize(
    "shape,with_bias,strided",
    [((256, 256, 256), True, False), ((64, 4096, 96), False, False), ((512, 4096, 512), True, True)],
    ids=["c1_bias", "k_heavy", "strided_lhs"],
)
def test_f32_split_k(device, oracle_mod, shape, with_bias, strided):
    """Small fp32 outputs with 32-aligned extents: one workgroup per 32 x 32 block sums K
    across its 16 waves (MFMA 32x32x2) and reduces the partial blocks in LDS. Shapes are
    (M, K, N): K = 4096 runs 16 slices per wave (the multi-slice loop), and the strided case
    has lhs row stride K + 8. Tolerance as in test_f32_matrix_core_shapes: the demo's
    rtol/atol plus 4 sqrt(K) 2^-24 (|A| |B|)."""

    import torch

    m, k, n = shape
    # the entry must route the shape to the split-K kernel (fewer than 32 tiles of 128 x 128
    # keep it off the fp32 MFMA GEMM): its cost record is the split-K MFMA count
    spec = [native.TensorSpec((m, n), "float32"), native.TensorSpec((m, k), "float32", (k + 8 if strided else k, 1)),
            native.TensorSpec((k, n), "float32"), native.TensorSpec((n,), "float32") if with_bias else None]
    assert ((m + 127) // 128) * ((n + 127) // 128) < 32
    assert native.cost("matmul", spec)["MFMA"] == (m // 32) * (n // 32) * (k // 16) * 8
    rng = np.random.default_rng(m + k + n)
    lhs = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    rhs = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = rng.uniform(-1, 1, n).astype(np.float32) if with_bias else None
    lt, rt = torch.from_numpy(lhs).to(device), torch.from_numpy(rhs).to(device)
    if strided:  # lhs row stride k + 8
        lt = torch.cat([lt, torch.zeros(m, 8, device=device)], 1)[:, :k]
    out = torch.full((m, n), float("nan"), device=device)
    print(f"[matmul] f32 split-K M={m} K={k} N={n} bias={with_bias} lda={lt.stride(0)}", flush=True)
    native.matmul(out, lt, rt, None if bias is None else torch.from_numpy(bias).to(device))
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, (64, 64, 64))
    terms = np.abs(lhs).astype(np.float64) @ np.abs(rhs).astype(np.float64)
    tol = 1e-4 * np.abs(ref) + 1e-5 + 4 * np.sqrt(k) * 2.0 ** -24 * terms
    err = np.abs(to_numpy(out).astype(np.float64) - ref)
    assert (err <= tol).all(), f"{shape}: max err/tol {np.max(err / tol):.3g}"


@pytest.mark.parametrize(
    "cfg",
    [
        ("C2", 4096, 4096, 4096, 20261202, [(0, 96), (2016, 2112), (4000, 4096)]),
        ("C2'", 8192, 4096, 1024, 20261203, [(0, 96), (8096, 8192)]),
    ],
    ids=["C2", "C2_skinny"],
)
def test_full_size_bf16(device, oracle_mod, cfg):
    """Full BASELINE shapes: sampled row blocks against the oracle (fp32 math on the
    bf16-rounded inputs) and a checksum-of-checksums over the whole output."""

    import torch

    name, m, k, n, seed, row_blocks = cfg
    rng = np.random.default_rng(seed)
    lt, lhs = round_to((rng.standard_normal((m, k), dtype=np.float32) * 0.02), torch.bfloat16)
    rt, rhs = round_to((rng.standard_normal((k, n), dtype=np.float32) * 0.02), torch.bfloat16)
    out = run(device, torch.bfloat16, lt, rt)
    got = to_numpy(out)
    for r0, r1 in row_blocks:
        ref = oracle_mod.matmul_demo(lhs[r0:r1], rhs, None, (48, 256, 256))
        assert_h16_close(got[r0:r1], ref, what=f"{name} rows {r0}:{r1}")
    # column sums of C equal (1^T A) B: a property of the whole product, checked in fp64
    colsum_ref = lhs.astype(np.float64).sum(0) @ rhs.astype(np.float64)
    colsum = got.astype(np.float64).sum(0)
    scale = np.sqrt(m) * np.abs(got).mean() + 1e-12
    assert np.max(np.abs(colsum - colsum_ref)) < 2e-2 * scale, name


def test_rejects_mismatched_shapes(device):
    import torch

    a = torch.zeros(4, 5, device=device)
    b = torch.zeros(6, 3, device=device)
    c = torch.zeros(4, 3, device=device)
    with pytest.raises(native.NativeLibraryError):
        native.matmul(c, a, b, None)
    with pytest.raises(native.NativeLibraryError):  # host memory is refused, not dereferenced
        native.matmul(torch.zeros(4, 3), torch.zeros(4, 6), torch.zeros(6, 3), None)
    # a slot whose shape claims more memory than its device allocation holds is refused
    lhs = torch.zeros(4, 8, device=device)
    rhs = torch.zeros(8, 3, device=device)
    slots, keep = native.marshal_slots((c, lhs, rhs, None))
    slots[1].shape[1] = 1 << 32
    slots[1].stride[0] = 1 << 32
    slots[2].shape[0] = 1 << 32
    lib = native.load_library()
    assert lib.kg_gfx950_matmul_entry(slots, 4) == -1
    assert "allocation" in native.last_error()


@pytest.mark.parametrize("shape", [(512, 256, 768), (2048, 1024, 8192)], ids=["tile128", "tile256"])
def test_memory_stage_depths_bit_identical(device, oracle_mod, shape):
    """Slot 7 (memory_stage 2/3/4) changes only the LDS ring depth of the pipelined kernel,
    not the order of any accumulation: every depth gives the default run's bits. Shapes
    cover both tile heights and K lengths with steady slices and tails at every depth."""

    import torch

    m, k, n = shape
    rng = np.random.default_rng(m + k + n)
    lt, lhs = round_to(rng.standard_normal((m, k), dtype=np.float32) * 0.05, torch.bfloat16)
    rt, rhs = round_to(rng.standard_normal((k, n), dtype=np.float32) * 0.05, torch.bfloat16)
    default = run(device, torch.bfloat16, lt, rt)
    a, b = lt.to(device), rt.to(device)
    for stages in (2, 3, 4):
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=device)
        print(f"[matmul] {shape} memory_stage={stages}", flush=True)
        native.call_entry("kg_gfx950_matmul_entry", (out, a, b, None, 64, 64, 64, stages))
        assert torch.equal(out, default), f"memory_stage={stages}"
    ref = oracle_mod.matmul_demo(lhs[:64], rhs, None, (64, 64, 64))
    assert_h16_close(to_numpy(default)[:64], ref, what=f"{shape} rows 0:64")
    with pytest.raises(native.NativeLibraryError, match="memory_stage"):
        native.call_entry("kg_gfx950_matmul_entry", (default, a, b, None, 64, 64, 64, 5))
