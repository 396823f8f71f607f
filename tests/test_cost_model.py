"""CPU tests of the gfx950 cost model: kg_gfx950_cost through native.cost and
tools.dsl_cost_run (contract of kernel_gen/tools/dsl_run.py:656-730, tests in
test/tools/test_dsl_cost_run.py: required cost_kind, kind and target checks, arity, int
result).

MAC and byte counts are pinned by brute force (an oracle run gives the output shape; a
mask count gives the causal pairs); MFMA counts are pinned by the MAC content of one
MFMA (16x16x32: 8192 MACs in the pipelined GEMM and the attention kernel; 32x32x16: 16384
in the conv kernels; fp32 32x32x2: 2048) on exact-tile shapes, and by the hardware counter
SQ_INSTS_MFMA on every kernel choice (profiles/mfma_instruction_counts.txt, made by
tests/cost_cases.py under rocprofv3 --pmc). MFMA_CYCLES is the MFMA count times 16, 32 or
64 by the same shapes.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd import native
from kernelcode_generate_amd.core.config import restore_config, set_target, snapshot_config
from kernelcode_generate_amd.core.error import KernelCodeError
from kernelcode_generate_amd.kernel.conv2d.inputs_dynamic_tile_dynamic import conv2d_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_static import conv2d_inputs_static_tile_static_kernel
from kernelcode_generate_amd.kernel.flash_attention.inputs_static_tile_static import (
    flash_attention_inputs_static_tile_static_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.scaled import (
    flash_attention_scaled_causal_kernel,
    flash_attention_scaled_kernel,
)
from kernelcode_generate_amd.kernel.matmul.inputs_dynamic_tile_dynamic import matmul_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_static import matmul_inputs_static_tile_static_kernel
from kernelcode_generate_amd.tools import VALID_DSL_COST_KINDS, dsl_cost_run
from tests.cost_cases import CASES, modelled

T = native.TensorSpec
PIPE = "gfx950-lowering"
MFMA_MACS = 32 * 32 * 16  # 16-bit conv kernels
GEMM_MFMA_MACS = 16 * 16 * 32  # pipelined 16-bit GEMM and 16-bit attention
PROFILE = Path(__file__).resolve().parents[1] / "profiles" / "mfma_instruction_counts.txt"


@pytest.fixture(autouse=True)
def gfx950_target():
    snap = snapshot_config()
    set_target("gfx950")
    yield
    restore_config(snap)


def costs(fn, args):
    return {kind: dsl_cost_run(fn, args, PIPE, kind) for kind in VALID_DSL_COST_KINDS}


def test_contract_checks():
    a = (T((8, 8), "float32"),) * 3 + (None, 8, 8, 8)
    with pytest.raises(KernelCodeError, match="DslCostRunInvalidCostKind"):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a, PIPE, "DMA1")
    with pytest.raises(TypeError):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a, PIPE)  # cost_kind has no default
    with pytest.raises(KernelCodeError, match="DslRunArityMismatch"):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a[:-1], PIPE, "MAC")
    with pytest.raises(KernelCodeError):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a, "no-such-pipeline", "MAC")
    set_target("npu_demo")
    with pytest.raises(KernelCodeError, match="DslCostRunInvalidTarget"):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a, PIPE, "MAC")
    set_target("gfx950")
    assert isinstance(dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, a, PIPE, "MAC"), int)


def test_entry_validation_applies():
    """A call the entry would reject is rejected by the cost query, with its message."""

    bad = (T((8, 8), "float32"), T((8, 4), "float32"), T((5, 8), "float32"), None, 8, 8, 8)
    with pytest.raises(KernelCodeError, match="DslCostRunInvalidOutput.*lhs K=4 != rhs K=5"):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, bad, PIPE, "MAC")
    mixed = (T((8, 8), "bfloat16"), T((8, 8), "float16"), T((8, 8), "bfloat16"), None, 8, 8, 8)
    with pytest.raises(KernelCodeError, match="dtypes must match"):
        dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, mixed, PIPE, "MFMA")
    qkv = (T((1, 1, 8, 16), "bfloat16"),) * 3
    with pytest.raises(native.NativeLibraryError, match="causal mask needs S_q == S_kv"):
        native.cost("flash_attention", [T((1, 1, 8, 16), "bfloat16"), qkv[0], T((1, 1, 9, 16), "bfloat16"),
                                        T((1, 1, 9, 16), "bfloat16"), 64, 64, 1.0, 1])
    with pytest.raises(native.NativeLibraryError, match="no cost model"):
        native.cost("softmax", [])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("mnk", [(4096, 4096, 4096), (512, 768, 256), (1000, 1000, 520), (7, 9, 3)])
def test_matmul_counts(dtype, mnk):
    m, n, k = mnk
    lhs, rhs, out = np.zeros((m, k), np.float32), np.zeros((k, n), np.float32), np.zeros((m, n), np.float32)
    args = (T(out.shape, dtype), T(lhs.shape, dtype), T(rhs.shape, dtype), T((n,), "float32"), 64, 64, 64)
    c = costs(matmul_inputs_dynamic_tile_dynamic_kernel, args)
    es = 4 if dtype == "float32" else 2
    assert c["MAC"] == out.size * k  # one multiply-add per (row, column, k)
    assert c["HBM_READ"] == (lhs.size + rhs.size) * es + n * 4  # fp32 bias
    assert c["HBM_WRITE"] == out.size * es
    if dtype == "float32":
        tiles = -(-m // 128) * -(-n // 128)
        if tiles >= 32 and k >= 64 and k % 4 == 0 and n % 4 == 0:  # fp32 MFMA: 32x32x2 = 2048 MACs each
            assert c["MFMA"] * 2048 >= c["MAC"]
            if m % 128 == 0 and n % 128 == 0 and k % 16 == 0:
                assert c["MFMA"] * 2048 == c["MAC"]
        elif m % 32 == 0 and n % 32 == 0 and k % 16 == 0:  # split-K blocks of 32 x 32: exact
            assert c["MFMA"] * 2048 == c["MAC"]
        else:
            assert c["MFMA"] == 0  # SIMT path
    elif k % 8 or n % 8:
        assert c["MFMA"] == 0  # SIMT path
    elif m % 256 == 0 and n % 256 == 0 and k % 64 == 0:
        assert c["MFMA"] * GEMM_MFMA_MACS == c["MAC"]  # exact tiles: no wasted MFMA work
    else:
        assert c["MFMA"] * GEMM_MFMA_MACS >= c["MAC"]
    # 1024 16-bit or 64 fp32 FLOP per SIMD cycle, whichever MFMA shape the kernel uses
    assert c["MFMA_CYCLES"] == c["MFMA"] * (64 if dtype == "float32" else 16)


def test_matmul_static_demo_uses_baked_tiles():
    args = (T((96, 80), "float32"), T((96, 56), "float32"), T((56, 80), "float32"), None)
    assert dsl_cost_run(matmul_inputs_static_tile_static_kernel, args, PIPE, "MAC") == 96 * 80 * 56
    assert dsl_cost_run(matmul_inputs_static_tile_static_kernel, args, PIPE, "HBM_READ") == (96 * 56 + 56 * 80) * 4


def test_conv_counts_match_oracle_shape(oracle_mod):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 5, 13, 11), dtype=np.float32)
    w = rng.standard_normal((4, 5, 3, 2), dtype=np.float32)
    stride, dil, pad = (2, 1), (1, 2), (1, 0, 2, 1)
    y = oracle_mod.conv2d_demo(x, w, None, stride, dil, pad, (4, 5, 2, 3, 3))
    args = (T(y.shape, "float32"), T(x.shape, "float32"), T(w.shape, "float32"), None, *stride, *dil, *pad, 4, 5, 2, 3, 3)
    c = costs(conv2d_inputs_dynamic_tile_dynamic_kernel, args)
    assert c["MAC"] == y.size * 5 * 3 * 2  # every output element sums C*KH*KW taps (padding included)
    assert c["HBM_READ"] == x.nbytes + w.nbytes and c["HBM_WRITE"] == y.nbytes
    # fp32 implicit GEMM: one 64 x 128 tile per 128 output pixels, 16-deep K slices, 4 waves x
    # 2 blocks x 8 MFMAs (32x32x2 = 2048 MACs each) per slice
    tiles = -(-y.shape[0] * y.shape[2] * y.shape[3] // 128)
    assert c["MFMA"] == tiles * -(-30 // 16) * 4 * 2 * 8 and c["MFMA"] * 2048 >= c["MAC"]
    with pytest.raises(KernelCodeError, match="out shape"):
        bad = (T((2, 4, 7, 6), "float32"),) + args[1:]
        dsl_cost_run(conv2d_inputs_dynamic_tile_dynamic_kernel, bad, PIPE, "MAC")


def test_conv_static_demo_forwards_baked_geometry(oracle_mod):
    """stride 8 and pads (3, 3, 4, 0) are baked into the static demo's entry: the cost query
    accepts only the output shape those constants give."""

    x = np.zeros((1, 3, 40, 33), np.float32)
    w = np.zeros((2, 3, 5, 3), np.float32)
    y = oracle_mod.conv2d_demo(x, w, None, (8, 8), (1, 1), (3, 3, 4, 0), (2, 3, 1, 2, 2))
    args = (T(y.shape, "float32"), T(x.shape, "float32"), T(w.shape, "float32"), None)
    assert dsl_cost_run(conv2d_inputs_static_tile_static_kernel, args, PIPE, "MAC") == y.size * 3 * 5 * 3


def test_conv_mfma_path():
    shape = (32, 64, 56, 56)
    args = (T(shape, "float16"), T(shape, "float16"), T((64, 64, 3, 3), "float16"), None, 1, 1, 1, 1, 1, 1, 1, 1,
            64, 64, 1, 7, 56)
    c = costs(conv2d_inputs_dynamic_tile_dynamic_kernel, args)
    assert c["MAC"] == 32 * 64 * 56 * 56 * 64 * 9
    # 56 columns fill 64 MFMA columns (two 32-wide waves): MFMA work is MAC * 64/56
    assert c["MFMA"] * MFMA_MACS * 56 == c["MAC"] * 64
    assert c["MFMA_CYCLES"] == 32 * c["MFMA"]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 2, 37, 16), (2, 1, 64, 8)])
def test_attention_macs_count_mask(shape, causal):
    b, h, s, d = shape
    kept = int(np.tril(np.ones((s, s))).sum()) if causal else s * s
    fn = flash_attention_scaled_causal_kernel if causal else flash_attention_scaled_kernel
    args = (T(shape, "float32"),) * 4 + (64, 64, 0.5)
    c = costs(fn, args)
    assert c["MAC"] == 2 * b * h * kept * d  # Q.K^T and P.V each take D multiply-adds per kept pair
    assert c["HBM_READ"] == 3 * b * h * s * d * 4 and c["HBM_WRITE"] == b * h * s * d * 4 and c["MFMA"] == 0


def test_attention_mfma_exact_tiles():
    """Exact tiles: the S^T and PV MFMAs (D/2 per wave and key tile) carry exactly the MACs;
    the kernel adds 4 row-sum MFMAs (P against ones) per wave and tile."""

    shape = (4, 32, 2048, 128)
    d = shape[3]
    c = costs(flash_attention_scaled_kernel, (T(shape, "bfloat16"),) * 4 + (128, 64, 0.088))
    assert c["MFMA"] * (d // 2) * GEMM_MFMA_MACS == c["MAC"] * (d // 2 + 4) and c["MFMA_CYCLES"] == 16 * c["MFMA"]
    static = costs(flash_attention_inputs_static_tile_static_kernel, (T(shape, "bfloat16"),) * 4)
    assert static["MAC"] == c["MAC"] and static["MFMA"] == c["MFMA"]


def test_attention_causal_mfma_bounds():
    """Causal blocks stop at their last query's key tile: MFMA work lies between the kept
    pairs and the full square."""

    shape = (1, 32, 16384, 128)
    d = shape[3]
    c = costs(flash_attention_scaled_causal_kernel, (T(shape, "bfloat16"),) * 4 + (128, 64, 0.088))
    full = 2 * 32 * 16384 * 16384 * 128
    assert c["MFMA"] % (d // 2 + 4) == 0
    product_mfma = c["MFMA"] // (d // 2 + 4) * (d // 2)  # without the 4 row-sum MFMAs per wave and tile
    assert c["MAC"] <= product_mfma * GEMM_MFMA_MACS < 0.51 * full


def _read_profile():
    rows = {}
    for line in PROFILE.read_text().splitlines():
        m = re.match(r"\|\s*(\w+)\s*\|\s*(\w+)\s*\|\s*(\d+)\s*\|\s*(\d+)\s*\|", line)
        if m:
            rows[m.group(1)] = (m.group(2), int(m.group(3)), int(m.group(4)))
    return rows


def test_mfma_model_matches_hardware_counter():
    rows = _read_profile()
    assert set(rows) == {case[0] for case in CASES}
    for case in CASES:
        kernel, counted, model_then = rows[case[0]]
        assert modelled(case)["MFMA"] == model_then == counted, case[0]


def test_roofline_kind():
    """ROOFLINE_NS: the larger of the MFMA time at the 2.4 GHz peak (16 cycles per 16-bit
    16x16x32 MFMA, 32 per 32x32x16, 64 per fp32 32x32x2, over 1024 SIMDs) and the compulsory
    bytes at 8 TB/s."""

    b16 = T((4096, 4096), "bfloat16")
    c2 = dsl_cost_run(matmul_inputs_dynamic_tile_dynamic_kernel, (b16, b16, b16, None, 64, 64, 64), PIPE, "ROOFLINE_NS")
    assert c2 == -(-8388608 * 16 // (1024 * 2.4)) == 54614  # 2 x 4096^3 FLOP at 2516.6 TFLOP/s
    x = T((32, 64, 56, 56), "float16")
    w = T((64, 64, 3, 3), "float16")
    conv = dsl_cost_run(conv2d_inputs_dynamic_tile_dynamic_kernel, (x, x, w, None) + (1,) * 8 + (8, 8, 8, 8, 8), PIPE,
                        "ROOFLINE_NS")
    mfma_ns = 258048 * 32 / 1024 / 2.4
    bytes_ns = (2 * 32 * 64 * 56 * 56 * 2 + 64 * 64 * 9 * 2) / 8000
    assert conv == int(-(-max(mfma_ns, bytes_ns) // 1))
