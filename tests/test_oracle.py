"""Pins the CPU oracle (oracle/kg_oracle.c) before it is trusted as the GPU checker.

Each oracle function is checked against something independent of its own text:
  - the known-answer values of the reference's tests (tests/golden/kat_primitives.npz,
    from test/include/api/test_kernel.py:199-364),
  - the reference's own npu_demo primitives compiled from its headers (oracle/_ref),
    element for element (skipped where that library was not built),
  - closed forms in float64 (np.matmul, pad+einsum conv, softmax attention) as used by
    the reference demos' own expected values (kernel/*/inputs_static_tile_static.py),
  - invariants the mathematics fixes (tile-size independence, causal row 0 = V[0],
    softmax rows sum to one, conv == implicit GEMM),
and a planted mistake in a copy of the inputs must make those checks fail.
"""

from __future__ import annotations

import random
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.golden.make_golden import attention_closed_form, conv_closed_form

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def kat():
    return dict(np.load(GOLDEN / "kat_primitives.npz"))


@pytest.fixture(scope="module")
def runtime_vectors():
    return dict(np.load(GOLDEN / "cuda_runtime_vectors.npz"))


@pytest.fixture(scope="module")
def ref():
    prims = oracle.reference_primitives()
    if prims is None:
        pytest.skip("oracle/_ref/libkg_npu_demo_ref.so not built (reference tree absent)")
    return prims


# --------------------------------------------------------------------------- KATs


def test_matmul_kat(kat):
    out = oracle.matmul(kat["matmul_lhs"], kat["matmul_rhs"])
    np.testing.assert_array_equal(out, kat["matmul_expected"])
    out2 = oracle.matmul(kat["matmul_lhs"], kat["matmul_rhs"], out=out, acc=True)
    np.testing.assert_array_equal(out2, kat["matmul_acc_expected"])


def test_reduce_max_kat(kat):
    np.testing.assert_array_equal(oracle.reduce_rows(kat["reduce_input"], "max"), kat["reduce_max_expected"])


def test_img2col2d_kat(kat):
    out = oracle.img2col2d(kat["img2col2d_input"], 2, 2, 1, 1, 1, 1, 0, 0, 0, 0)
    np.testing.assert_array_equal(out, kat["img2col2d_expected"])


def test_exp_kat(kat):
    x = kat["exp_input"]
    out = oracle.exp(x)
    # test_kernel.py:285-288 bounds: |exp(1)-e| <= 1e-4, |exp(6)| within 1e-2
    assert abs(out[0, 0] - np.exp(np.float32(1.0))) <= 1e-4
    assert abs(out[1, 2] - np.exp(np.float32(6.0))) <= 1e-2
    np.testing.assert_array_equal(out, np.exp(x.astype(np.float64)).astype(np.float32))


# ------------------------------------------------- the reference's own primitives


@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 3, 4), (37, 53, 29), (64, 80, 48)])
def test_matmul_matches_reference_primitive(ref, shape):
    m, k, n = shape
    rng = np.random.default_rng(sum(shape))
    a = rng.normal(size=(m, k)).astype(np.float32)
    b = rng.normal(size=(k, n)).astype(np.float32)
    c = rng.normal(size=(m, n)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, b), ref.matmul(a, b))
    np.testing.assert_array_equal(oracle.matmul(a, b, out=c, acc=True), ref.matmul(a, b, out=c, acc=True))


@pytest.mark.parametrize(
    "args",
    [
        (3, 3, 1, 1, 1, 1, 1, 1, 1, 1),
        (3, 5, 8, 8, 1, 1, 3, 3, 4, 0),
        (2, 2, 8, 8, 1, 1, 4, 3, 4, 3),
        (5, 3, 2, 3, 2, 1, 0, 4, 2, 1),
    ],
)
def test_img2col2d_matches_reference_primitive(ref, args):
    rng = np.random.default_rng(7)
    x = rng.normal(size=(2, 3, 19, 23)).astype(np.float32)
    np.testing.assert_array_equal(oracle.img2col2d(x, *args), ref.img2col2d(x, *args))


def test_exp_reduce_match_reference_primitives(ref):
    rng = np.random.default_rng(11)
    x = (rng.normal(size=(7, 33)) * 8).astype(np.float32)
    x[0, :5] = -np.inf
    np.testing.assert_array_equal(oracle.exp(x), ref.exp(x))
    np.testing.assert_array_equal(oracle.reduce_rows(x, "max"), ref.reduce_rows(x, "max"))
    np.testing.assert_array_equal(oracle.reduce_rows(x, "sum"), ref.reduce_rows(x, "sum"))


def test_binary_ops_of_fa_update_match_reference(ref):
    # the online-softmax state update uses max, sub, mul, add, truediv (Kernel.h:284-443)
    rng = np.random.default_rng(3)
    a = rng.normal(size=(4, 9)).astype(np.float32)
    b = rng.normal(size=(4, 9)).astype(np.float32) + 3
    np.testing.assert_array_equal(ref.binary(a, b, "max"), np.where(a > b, a, b))
    np.testing.assert_array_equal(ref.binary(a, b, "truediv"), (a.astype(np.float64) / b).astype(np.float32))
    np.testing.assert_array_equal(ref.binary(a, b, "sub"), a - b)
    np.testing.assert_array_equal(ref.binary(a, b, "mul"), a * b)
    np.testing.assert_array_equal(ref.binary(a, b, "add"), a + b)


# ------------------------------------------------------------ reference runtime vectors


def test_matmul_demo_runtime_vectors(runtime_vectors):
    v = runtime_vectors
    np.testing.assert_array_equal(oracle.matmul_demo(v["matmul_lhs"], v["matmul_rhs"], None, (2, 2, 2)), v["matmul_absent"])
    np.testing.assert_array_equal(
        oracle.matmul_demo(v["matmul_lhs"], v["matmul_rhs"], v["matmul_bias"], (2, 2, 2)), v["matmul_present"]
    )


@pytest.mark.parametrize("case", [0, 1])
def test_conv2d_demo_runtime_vectors(runtime_vectors, case):
    p = runtime_vectors[f"conv{case}_params"]
    xs, ws, stride, dil, pad = tuple(p[0:4]), tuple(p[4:8]), tuple(p[8:10]), tuple(p[10:12]), tuple(p[12:16])
    x = np.arange(int(np.prod(xs)), dtype=np.float32).reshape(xs)
    w = np.arange(int(np.prod(ws)), dtype=np.float32).reshape(ws) / np.float32(7.0)
    b = np.arange(ws[0], dtype=np.float32)
    for tiles in [(7, 18, 3, 9, 8), (1, 1, 1, 1, 1)]:
        out = oracle.conv2d_demo(x, w, None, stride, dil, pad, tiles)
        np.testing.assert_allclose(out, runtime_vectors[f"conv{case}_absent"], rtol=1e-5, atol=1e-5)
        out = oracle.conv2d_demo(x, w, b, stride, dil, pad, tiles)
        np.testing.assert_allclose(out, runtime_vectors[f"conv{case}_present"], rtol=1e-5, atol=1e-5)


def test_flash_attention_demo_runtime_vector(runtime_vectors):
    v = runtime_vectors
    for br, bc in [(2, 2), (4, 4), (3, 1)]:
        out = oracle.flash_attention_demo(v["fa_q"], v["fa_k"], v["fa_v"], br, bc)
        np.testing.assert_allclose(out, v["fa_expected"], rtol=1e-4, atol=1e-4)


# -------------------------------------------------------------------- closed forms


def _demo_matmul_shape():
    # module-level static shape of kernel/matmul/inputs_static_tile_static.py:50-57
    rng = random.Random(2026051601)
    m, k, n = rng.randint(160, 256), rng.randint(160, 256), rng.randint(160, 256)
    tiles = random.Random(2026051700).choice(((72, 56, 48), (48, 80, 56)))
    return m, k, n, tiles


@pytest.mark.parametrize("fused", [True, False])
def test_matmul_demo_closed_form(fused):
    m, k, n, tiles = _demo_matmul_shape()
    # the demo's annotation defaults: out [166, 172], lhs [166, 217] (inputs_static_tile_static.py:61-63)
    assert (m, k, n) == (166, 217, 172)
    rng = np.random.default_rng(2026051601)
    lhs = rng.normal(size=(m, k)).astype(np.float32)
    rhs = rng.normal(size=(k, n)).astype(np.float32)
    bias = rng.normal(size=(n,)).astype(np.float32)
    exp = lhs.astype(np.float64) @ rhs
    for tl in (tiles, (48, 80, 56), (256, 256, 256), (1, 7, 3)):
        np.testing.assert_allclose(oracle.matmul_demo(lhs, rhs, None, tl, fused=fused), exp, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(oracle.matmul_demo(lhs, rhs, bias, tl, fused=fused), exp + bias, rtol=1e-4, atol=1e-4)


def test_matmul_demo_fused_is_sequential_k():
    # with K-loop fusion the result equals one sequential-k pass over the whole K,
    # i.e. is independent of tile_k bit for bit
    rng = np.random.default_rng(5)
    lhs = rng.normal(size=(33, 70)).astype(np.float32)
    rhs = rng.normal(size=(70, 21)).astype(np.float32)
    full = oracle.matmul(lhs, rhs)
    for tk in (1, 7, 48, 70, 128):
        np.testing.assert_array_equal(oracle.matmul_demo(lhs, rhs, None, (16, 8, tk)), full)


@pytest.mark.parametrize(
    "xs,ws,stride,dil,pad,tiles",
    [
        ((3, 20, 57, 45), (11, 20, 3, 5), (8, 8), (1, 1), (3, 3, 4, 0), (8, 16, 4, 8, 9)),
        ((2, 9, 30, 31), (5, 9, 3, 3), (1, 1), (1, 1), (1, 1, 1, 1), (7, 18, 3, 9, 8)),
        ((2, 6, 29, 23), (4, 6, 2, 3), (2, 3), (2, 1), (0, 4, 2, 1), (6, 20, 2, 10, 7)),
        ((1, 4, 5, 7), (3, 4, 5, 3), (1, 2), (1, 1), (2, 2, 0, 1), (1, 1, 1, 1, 1)),
    ],
)
def test_conv2d_demo_closed_form(xs, ws, stride, dil, pad, tiles):
    rng = np.random.default_rng(len(xs) + ws[0])
    x = rng.normal(size=xs).astype(np.float32)
    w = rng.normal(size=ws).astype(np.float32)
    b = rng.normal(size=(ws[0],)).astype(np.float32)
    np.testing.assert_allclose(
        oracle.conv2d_demo(x, w, b, stride, dil, pad, tiles), conv_closed_form(x, w, b, stride, dil, pad), rtol=1e-4, atol=1e-4
    )


def test_conv2d_is_implicit_gemm():
    # conv == W[F, C*KH*KW] @ img2col(x)[C*KH*KW, Ho*Wo] per image (K order c, kh, kw)
    rng = np.random.default_rng(9)
    x = rng.normal(size=(1, 5, 12, 10)).astype(np.float32)
    w = rng.normal(size=(4, 5, 3, 3)).astype(np.float32)
    col = oracle.img2col2d(x, 3, 3, 1, 1, 1, 1, 1, 1, 1, 1)
    gemm = oracle.matmul(w.reshape(4, -1), col.reshape(45, -1)).reshape(1, 4, 12, 10)
    np.testing.assert_allclose(oracle.conv2d_demo(x, w, None, (1, 1), (1, 1), (1, 1, 1, 1), (4, 5, 1, 12, 10)), gemm,
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize(
    "shape,br,bc,scale,causal",
    [
        ((1, 2, 4, 3), 2, 2, None, False),
        ((2, 3, 257, 48), 48, 64, None, False),
        ((1, 2, 321, 64), 64, 80, None, False),
        ((1, 1, 389, 80), 80, 96, None, False),
        ((1, 2, 256, 64), 64, 64, 0.125, True),
        ((1, 1, 200, 32), 48, 80, 0.3, True),
    ],
)
def test_flash_attention_demo_closed_form(shape, br, bc, scale, causal):
    rng = np.random.default_rng(shape[2])
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
    out = oracle.flash_attention_demo(q, k, v, br, bc, scale=scale, causal=causal)
    exp = attention_closed_form(q, k, v, 1.0 if scale is None else scale, causal)
    np.testing.assert_allclose(out, exp, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------------- invariants


def test_flash_attention_invariants():
    rng = np.random.default_rng(21)
    q, k, v = (rng.standard_normal((1, 2, 96, 16), dtype=np.float32) for _ in range(3))
    a = oracle.flash_attention_demo(q, k, v, 32, 32, causal=True)
    b = oracle.flash_attention_demo(q, k, v, 48, 16, causal=True)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5)  # tile-size independence
    np.testing.assert_allclose(a[:, :, 0, :], v[:, :, 0, :], rtol=1e-6, atol=1e-6)  # causal row 0 = V[0]
    ones = np.ones_like(v)
    np.testing.assert_allclose(oracle.flash_attention_demo(q, k, ones, 32, 24), ones, rtol=1e-5, atol=1e-5)  # rows sum to 1


def test_planted_mistakes_are_caught():
    """A dropped term, a transposed operand or a wrong sign in the inputs must fail the checks."""

    rng = np.random.default_rng(13)
    lhs = rng.normal(size=(20, 24)).astype(np.float32)
    rhs = rng.normal(size=(24, 24)).astype(np.float32)
    good = oracle.matmul_demo(lhs, rhs, None, (8, 8, 8))
    exp = lhs.astype(np.float64) @ rhs
    assert np.allclose(good, exp, rtol=1e-4, atol=1e-4)
    dropped = lhs.copy()
    dropped[:, -1] = 0  # drop the last k term
    assert not np.allclose(oracle.matmul_demo(dropped, rhs, None, (8, 8, 8)), exp, rtol=1e-4, atol=1e-4)
    assert not np.allclose(oracle.matmul_demo(lhs, rhs.T.copy(), None, (8, 8, 8)), exp, rtol=1e-4, atol=1e-4)
    q, k, v = (rng.standard_normal((1, 1, 40, 8), dtype=np.float32) for _ in range(3))
    ref = attention_closed_form(q, k, v, 0.5, False)
    assert np.allclose(oracle.flash_attention_demo(q, k, v, 16, 16, scale=0.5), ref, rtol=1e-4, atol=1e-4)
    assert not np.allclose(oracle.flash_attention_demo(q, k, v, 16, 16, scale=-0.5), ref, rtol=1e-4, atol=1e-4)
    assert not np.allclose(oracle.flash_attention_demo(q, k, v, 16, 16, scale=0.5, causal=True), ref, rtol=1e-4, atol=1e-4)
