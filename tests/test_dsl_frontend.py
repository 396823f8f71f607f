"""CPU tests of the DSL front end (dsl.mlir_gen), the passes (kernel-aggregate,
kernel-pattern-fuse) and the per-operation emitter.

The demo kernels are DSL programs (kernel/*); their IR, executed by a numpy interpreter
of the per-operation semantics (tests/ir_interp.py), must reproduce the oracle's
restatement of the reference's loop nests bit for bit in fp32 -- which pins what the front
end and kernel-aggregate produce. Pattern recognition must find each family by structure
and index arithmetic: a renamed kernel with renamed parameters still fuses, and a kernel
whose arithmetic differs in one place does not.
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from kernelcode_generate_amd.core.error import KernelCodeError
from kernelcode_generate_amd.dsl import mlir_gen
from kernelcode_generate_amd.ir import Cmp, format_func
from kernelcode_generate_amd.kernel.conv2d import inputs_static_tile_static as conv_static
from kernelcode_generate_amd.kernel.conv2d.inputs_dynamic_tile_dynamic import conv2d_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.conv2d.inputs_static_tile_dynamic import conv2d_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.flash_attention import inputs_static_tile_static as fa_static
from kernelcode_generate_amd.kernel.flash_attention.inputs_dynamic_tile_dynamic import (
    flash_attention_inputs_dynamic_tile_dynamic_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.inputs_static_tile_dynamic import (
    flash_attention_inputs_static_tile_dynamic_kernel,
)
from kernelcode_generate_amd.kernel.flash_attention.scaled import (
    flash_attention_scaled_causal_kernel,
    flash_attention_scaled_kernel,
)
from kernelcode_generate_amd.kernel.matmul import inputs_static_tile_static as mm_static
from kernelcode_generate_amd.kernel.matmul.inputs_dynamic_tile_dynamic import matmul_inputs_dynamic_tile_dynamic_kernel
from kernelcode_generate_amd.kernel.matmul.inputs_static_tile_dynamic import matmul_inputs_static_tile_dynamic_kernel
from kernelcode_generate_amd.operation import kernel
from kernelcode_generate_amd.operation.dma import alloc, broadcast, deslice, fill, reshape, view
from kernelcode_generate_amd.operation.scf import loop
from kernelcode_generate_amd.passes import kernel_aggregate, pattern_fuse
from kernelcode_generate_amd.pipeline import get_pipeline
from kernelcode_generate_amd.symbol_variable import MemorySpace, NumericType, SymbolDim
from tests import ir_interp


def lowered(fn, args, fuse=True):
    return get_pipeline("gfx950-lowering", {"fuse": fuse}).run(mlir_gen(fn, args))


def run_ir(fn, args, out_index=0):
    lw = lowered(fn, args, fuse=False)
    ir_interp.run(lw.func, args)
    return args[out_index]


# ------------------------------------------------------------------------------------
# front end + kernel-aggregate against the oracle (fp32, bit for bit)
# ------------------------------------------------------------------------------------


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("variant", ["static", "static_dyn", "dyn"])
def test_matmul_demo_ir_matches_oracle(oracle_mod, variant, with_bias):
    rng = np.random.default_rng(11)
    m, k, n = 97, 130, 75
    lhs = rng.standard_normal((m, k), dtype=np.float32)
    rhs = rng.standard_normal((k, n), dtype=np.float32)
    bias = rng.standard_normal(n, dtype=np.float32) if with_bias else None
    out = np.zeros((m, n), np.float32)
    if variant == "static":
        fn, extra, tiles = mm_static.matmul_inputs_static_tile_static_kernel, (), (mm_static._TILE_M, mm_static._TILE_N,
                                                                                  mm_static._TILE_K)
    elif variant == "static_dyn":
        fn, extra, tiles = matmul_inputs_static_tile_dynamic_kernel, (32, 24, 40), (32, 24, 40)
    else:
        fn, extra, tiles = matmul_inputs_dynamic_tile_dynamic_kernel, (50, 64, 17), (50, 64, 17)
    got = run_ir(fn, (out, lhs, rhs, bias, *extra))
    ref = oracle_mod.matmul_demo(lhs, rhs, bias, tiles)
    assert np.array_equal(got, ref)


def test_kernel_aggregate_folds_only_the_k_loop():
    a = np.zeros((8, 8), np.float32)
    func = mlir_gen(matmul_inputs_static_tile_dynamic_kernel, (a, a, a, None, 4, 4, 4))
    assert kernel_aggregate(func) == 1
    mm = [op for op in func.walk() if op.name == "kernel.matmul"][0]
    assert isinstance(mm.attrs["acc"], Cmp) and mm.attrs["acc"].op == "ne"
    assert mm.operands[0].name == "acc"
    assert not any(op.name == "kernel.binary_elewise" and op.operands[2].name == "partial" for op in func.walk())
    x = np.zeros((1, 2, 6, 6), np.float32)
    conv = mlir_gen(conv2d_inputs_static_tile_dynamic_kernel, (x, x, x, None, 2, 2, 1, 2, 2))
    assert kernel_aggregate(conv) == 0  # the conv product is transposed before it is added
    fa = mlir_gen(flash_attention_inputs_static_tile_dynamic_kernel, (x, x, x, x, 2, 2))
    assert kernel_aggregate(fa) == 0


@pytest.mark.parametrize("variant", ["static", "static_dyn", "dyn"])
def test_conv_demo_ir_matches_oracle(oracle_mod, variant):
    rng = np.random.default_rng(5)
    if variant == "static":
        fn = conv_static.conv2d_inputs_static_tile_static_kernel
        stride = (8, 8)
        pads = (conv_static._STATIC_PAD_TOP, conv_static._STATIC_PAD_BOTTOM, conv_static._STATIC_PAD_LEFT,
                conv_static._STATIC_PAD_RIGHT)
        dil = (1, 1)
        xs, ws = (2, 5, 37, 29), (6, 5, 3, 5)
        tiles = (conv_static._STATIC_TILE_F, conv_static._STATIC_TILE_C, conv_static._STATIC_TILE_N,
                 conv_static._STATIC_TILE_HO, conv_static._STATIC_TILE_WO)
        extra = ()
    elif variant == "static_dyn":
        from kernelcode_generate_amd.kernel.conv2d import inputs_static_tile_dynamic as mod

        fn = conv2d_inputs_static_tile_dynamic_kernel
        stride, dil = (8, 8), (1, 1)
        pads = (mod._STATIC_PAD_TOP, mod._STATIC_PAD_BOTTOM, mod._STATIC_PAD_LEFT, mod._STATIC_PAD_RIGHT)
        xs, ws = (3, 4, 30, 41), (5, 4, 3, 3)
        tiles = (2, 3, 2, 2, 3)
        extra = tiles
    else:
        fn = conv2d_inputs_dynamic_tile_dynamic_kernel
        stride, dil, pads = (2, 1), (1, 2), (1, 2, 0, 3)
        xs, ws = (2, 3, 11, 13), (4, 3, 3, 2)
        tiles = (3, 2, 1, 4, 5)
        extra = stride + dil + pads + tiles
    x = rng.standard_normal(xs, dtype=np.float32)
    w = rng.standard_normal(ws, dtype=np.float32)
    b = rng.standard_normal(ws[0], dtype=np.float32)
    ho, wo = oracle_mod.conv2d_out_hw(xs[2], xs[3], ws[2], ws[3], stride, dil, pads)
    for bias in (None, b):
        out = np.zeros((xs[0], ws[0], ho, wo), np.float32)
        got = run_ir(fn, (out, x, w, bias, *extra))
        ref = oracle_mod.conv2d_demo(x, w, bias, stride, dil, pads, tiles)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("variant", ["static", "static_dyn", "dyn", "scaled", "causal"])
def test_flash_attention_demo_ir_matches_oracle(oracle_mod, variant):
    rng = np.random.default_rng(3)
    shape = (1, 2, 45, 12)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
    out = np.zeros(shape, np.float32)
    scale, causal = None, False
    if variant == "static":
        fn, extra, tiles = fa_static.flash_attention_inputs_static_tile_static_kernel, (), (fa_static._STATIC_BR,
                                                                                           fa_static._STATIC_BC)
    elif variant == "static_dyn":
        fn, extra, tiles = flash_attention_inputs_static_tile_dynamic_kernel, (16, 10), (16, 10)
    elif variant == "dyn":
        fn, extra, tiles = flash_attention_inputs_dynamic_tile_dynamic_kernel, (7, 12), (7, 12)
    elif variant == "scaled":
        scale = 0.37
        fn, extra, tiles = flash_attention_scaled_kernel, (8, 16, scale), (8, 16)
    else:
        scale, causal = 0.29, True
        fn, extra, tiles = flash_attention_scaled_causal_kernel, (12, 5, scale), (12, 5)
    got = run_ir(fn, (out, q, k, v, *extra))
    ref = oracle_mod.flash_attention_demo(q, k, v, *tiles, scale=scale, causal=causal)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------------------------
# recognition by structure and index arithmetic
# ------------------------------------------------------------------------------------


def my_gemm(c: "Tensor[f32, M, N]", a: "Tensor[f32, M, K]", b: "Tensor[f32, K, N]", row_bias: "Tensor[f32, N]",
            bm: SymbolDim, bn: SymbolDim, bk: SymbolDim) -> None:
    rows, depth = a.get_shape()
    cols = b.get_shape()[1]
    for j0 in loop(0, cols, bn):  # column tiles outside, row tiles inside
        for i0 in loop(0, rows, bm):
            h = min(bm, rows - i0)
            w = min(bn, cols - j0)
            total = alloc([h, w], NumericType.Float32, MemorySpace.TSM)
            fill(total, 0)
            bias_tile = alloc([w], NumericType.Float32, MemorySpace.TSM)
            bias_plane = alloc([h, w], NumericType.Float32, MemorySpace.TSM)
            for p0 in loop(0, depth, bk):
                d = min(bk, depth - p0)
                ta = alloc([h, d], NumericType.Float32, MemorySpace.TSM)
                tb = alloc([d, w], NumericType.Float32, MemorySpace.TSM)
                fill(ta, 0)
                fill(tb, 0)
                deslice(ta, view(a, [i0, p0], [h, d], [1, 1]), [0, 0], [h, d], [1, 1])
                deslice(tb, view(b, [p0, j0], [d, w], [1, 1]), [0, 0], [d, w], [1, 1])
                prod = alloc([h, w], NumericType.Float32, MemorySpace.TSM)
                kernel.matmul(prod, ta, tb)
                kernel.add(total, total, prod)
            if row_bias is not None:
                deslice(bias_tile, view(row_bias, [j0], [w], [1]), [0], [w], [1])
                broadcast(bias_plane, reshape(bias_tile, [1, w]))
                kernel.add(total, total, bias_plane)
            deslice(c, total, [i0, j0], [h, w], [1, 1])


def my_gemm_wrong_offset(c: "Tensor[f32, M, N]", a: "Tensor[f32, M, K]", b: "Tensor[f32, K, N]", bm: SymbolDim,
                         bn: SymbolDim, bk: SymbolDim) -> None:
    rows, depth = a.get_shape()
    cols = b.get_shape()[1]
    for i0 in loop(0, rows, bm):
        for j0 in loop(0, cols, bn):
            h = min(bm, rows - i0)
            w = min(bn, cols - j0)
            total = alloc([h, w], NumericType.Float32, MemorySpace.TSM)
            fill(total, 0)
            for p0 in loop(0, depth, bk):
                d = min(bk, depth - p0)
                ta = alloc([h, d], NumericType.Float32, MemorySpace.TSM)
                tb = alloc([d, w], NumericType.Float32, MemorySpace.TSM)
                fill(ta, 0)
                fill(tb, 0)
                deslice(ta, view(a, [i0, p0], [h, d], [1, 1]), [0, 0], [h, d], [1, 1])
                # B's rows start half a tile late: not a matmul of a and b
                deslice(tb, view(b, [p0 + d // 2, j0], [d, w], [1, 1]), [0, 0], [d, w], [1, 1])
                prod = alloc([h, w], NumericType.Float32, MemorySpace.TSM)
                kernel.matmul(prod, ta, tb)
                kernel.add(total, total, prod)
            deslice(c, total, [i0, j0], [h, w], [1, 1])


def test_renamed_kernel_fuses_and_matches_oracle(oracle_mod):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((33, 50), dtype=np.float32)
    b = rng.standard_normal((50, 41), dtype=np.float32)
    bias = rng.standard_normal(41, dtype=np.float32)
    c = np.zeros((33, 41), np.float32)
    lw = lowered(my_gemm, (c, a, b, bias, 8, 16, 7))
    assert lw.fused is not None and lw.fused.family == "matmul"
    assert lw.fused.memory == ("c", "a", "b", "row_bias")
    got = run_ir(my_gemm, (c, a, b, bias, 8, 16, 7))
    assert np.array_equal(got, oracle_mod.matmul_demo(a, b, bias, (8, 16, 7)))


def test_different_index_arithmetic_does_not_fuse():
    a = np.zeros((16, 16), np.float32)
    lw = lowered(my_gemm_wrong_offset, (a, a, a, 4, 4, 4))
    assert lw.fused is None


def _mutate_source(fn, old: str, new: str):
    """A copy of the demo `fn` whose source has one edit (compiled in the demo's module)."""

    import inspect
    import textwrap
    import types

    src = textwrap.dedent(inspect.getsource(fn))
    assert old in src
    src = src.replace(old, new, 1).replace(f"def {fn.__name__}(", "def mutated_kernel(", 1)
    namespace = dict(fn.__globals__)
    code = compile(src, f"<mutated {fn.__name__}>", "exec")
    exec(code, namespace)
    mutated = namespace["mutated_kernel"]
    # inspect.getsource cannot see exec'd text: keep it on the function for the front end
    import linecache

    filename = f"<mutated {fn.__name__} {random.random()}>"
    linecache.cache[filename] = (len(src), None, src.splitlines(True), filename)
    mutated.__code__ = mutated.__code__.replace(co_filename=filename)
    assert isinstance(mutated, types.FunctionType)
    return mutated


@pytest.mark.parametrize(
    "old,new",
    [
        ("kernel.sub(shifted_score, score_tile, m_next_full)", "kernel.sub(shifted_score, m_next_full, score_tile)"),
        ('fill(m_state, "-inf")', "fill(m_state, 0)"),
        ("kernel.add(sum_next, scaled_sum, tile_sum)", "kernel.mul(sum_next, scaled_sum, tile_sum)"),
        ("v_4d = view(v, [b0, h0, n0, 0]", "v_4d = view(k, [b0, h0, n0, 0]"),
        ("for n0 in loop(0, seq_len, bc):", "for n0 in loop(0, seq_len - 1, bc):"),
    ],
)
def test_attention_mutations_do_not_fuse(old, new):
    x = np.zeros((1, 2, 16, 8), np.float32)
    args = (x, x, x, x, 4, 4)
    assert lowered(flash_attention_inputs_dynamic_tile_dynamic_kernel, args).fused is not None
    mutated = _mutate_source(flash_attention_inputs_dynamic_tile_dynamic_kernel, old, new)
    assert lowered(mutated, args).fused is None


@pytest.mark.parametrize(
    "old,new",
    [
        ("local_pad_top = max(pad_top - ho0 * stride_h, 0)", "local_pad_top = max(pad_top - ho0 * stride_h, 1)"),
        ("partial = transpose(out_fnhw, [1, 0, 2, 3])", "partial = transpose(out_fnhw, [1, 0, 3, 2])"),
        ("weight_tile = slice(weight, [f0, c0, 0, 0]", "weight_tile = slice(weight, [f0, 0, 0, 0]"),
    ],
)
def test_conv_mutations_do_not_fuse(old, new):
    x = np.zeros((1, 2, 9, 9), np.float32)
    w = np.zeros((2, 2, 3, 3), np.float32)
    args = (x, x, w, None, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 1, 3, 3)
    assert lowered(conv2d_inputs_dynamic_tile_dynamic_kernel, args).fused is not None
    mutated = _mutate_source(conv2d_inputs_dynamic_tile_dynamic_kernel, old, new)
    assert lowered(mutated, args).fused is None


def test_causal_form_is_recognised_from_the_row_mask():
    x = np.zeros((1, 1, 16, 8), np.float32)
    fused = lowered(flash_attention_scaled_causal_kernel, (x, x, x, x, 4, 4, 0.5)).fused
    assert fused.trailing_ints[0].value == 1 and fused.floats[0].arg == "scale"
    plain = lowered(flash_attention_scaled_kernel, (x, x, x, x, 4, 4, 0.5)).fused
    assert plain.trailing_ints[0].value == 0
    # a row mask that keeps one key too many is not causal attention
    wrong = _mutate_source(flash_attention_scaled_causal_kernel, "m0 + r + 1 - n0", "m0 + r + 2 - n0")
    assert lowered(wrong, (x, x, x, x, 4, 4, 0.5)).fused is None


# ------------------------------------------------------------------------------------
# front-end errors and the IR text
# ------------------------------------------------------------------------------------


def test_front_end_rejects_unsupported_constructs():
    def bad_loop(out: "Tensor[f32, N]") -> None:
        for i in range(3):  # Python range is not a DSL loop
            fill(out, 0)

    def bad_call(out: "Tensor[f32, N]") -> None:
        print(out)

    a = np.zeros(4, np.float32)
    for fn in (bad_loop, bad_call):
        with pytest.raises(KernelCodeError, match="mlir_gen"):
            mlir_gen(fn, (a,))
    with pytest.raises(KernelCodeError, match="positional"):
        mlir_gen(bad_loop, (a, a))


def test_ir_text_names_every_operation():
    x = np.zeros((1, 1, 8, 4), np.float32)
    text = format_func(mlir_gen(flash_attention_scaled_causal_kernel, (x, x, x, x, 4, 4, 0.5)))
    for name in ("symbol.for", "dma.alloc", "dma.fill", "dma.view", "dma.deslice", "dma.reshape", "dma.transpose",
                 "dma.broadcast", "kernel.matmul", "kernel.reduce", "kernel.exp", "kernel.binary_elewise"):
        assert name in text
    assert "present(" not in text and "scale" in text


def test_pattern_fuse_entry_point():
    a = np.zeros((8, 8), np.float32)
    func = mlir_gen(matmul_inputs_dynamic_tile_dynamic_kernel, (a, a, a, None, 4, 4, 4))
    assert pattern_fuse(func) is None  # before kernel-aggregate the K loop is not an accumulation
    kernel_aggregate(func)
    assert pattern_fuse(func).family == "matmul"
