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
from kernelcode_generate_amd.kernel.conv2d.tiled import tiled_conv2d
from kernelcode_generate_amd.kernel.flash_attention.tiled import online_softmax_attention
from kernelcode_generate_amd.kernel.matmul.tiled import tiled_matmul
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
    # a product-then-add K loop folds into one accumulating matmul
    func = mlir_gen(my_gemm, (a, a, a, None, 4, 4, 4))
    assert kernel_aggregate(func) == 1
    mm = [op for op in func.walk() if op.name == "kernel.matmul"][0]
    assert isinstance(mm.attrs["acc"], Cmp) and mm.attrs["acc"].op == "ne"
    assert mm.operands[0].name == "total"
    assert not any(op.name == "kernel.binary_elewise" and op.operands[2].name == "prod" for op in func.walk())
    # the matmul demos accumulate already; the conv product is added per channel tile and the
    # attention products are not K-loop sums: nothing to fold
    demo = mlir_gen(matmul_inputs_static_tile_dynamic_kernel, (a, a, a, None, 4, 4, 4))
    assert kernel_aggregate(demo) == 0
    x = np.zeros((1, 2, 6, 6), np.float32)
    conv = mlir_gen(conv2d_inputs_static_tile_dynamic_kernel, (x, x, x, None, 2, 2, 1, 2, 2))
    assert kernel_aggregate(conv) == 0
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


def _attention_kernel(helper, causal: bool):
    def attention(out: "Tensor[f32, B, H, S, D]", q: "Tensor[f32, B, H, S, D]", k: "Tensor[f32, B, H, S, D]",
                  v: "Tensor[f32, B, H, S, D]", br: SymbolDim, bc: SymbolDim, scale: float) -> None:
        helper(out, q, k, v, br, bc, scale, causal)

    return attention


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize(
    "old,new",
    [
        ("kernel.sub(probs, scores, probs)", "kernel.sub(probs, probs, scores)"),
        ('fill(run_max, "-inf")', "fill(run_max, 0)"),
        ("kernel.add(run_sum, run_sum, row_sum)", "kernel.mul(run_sum, run_sum, row_sum)"),
        ("v_rows = reshape(load(v,", "v_rows = reshape(load(k,"),
        ("for k0 in loop(0, kv_end, bc):", "for k0 in loop(0, kv_end - 1, bc):"),
        ("k_rows = reshape(load(k, [b, h, k0, 0]", "k_rows = reshape(load(k, [b, h, 0, 0]"),
        ("q_rows = reshape(load(q, [b, h, q0, 0]", "q_rows = reshape(load(q, [b, 0, q0, 0]"),
        ("kernel.exp(decay, decay)", "kernel.exp(decay, run_max)"),
        ("store(run_max, new_max, [0, 0], [nq, 1])", "store(run_max, tile_max, [0, 0], [nq, 1])"),
        ("kernel.truediv(o_acc, o_acc, denom)", "kernel.mul(o_acc, o_acc, denom)"),
    ],
)
def test_attention_mutations_do_not_fuse(old, new, causal):
    x = np.zeros((1, 2, 16, 8), np.float32)
    args = (x, x, x, x, 4, 4, 0.5)
    assert lowered(_attention_kernel(online_softmax_attention, causal), args).fused is not None
    mutated = _mutate_source(online_softmax_attention, old, new)
    assert lowered(_attention_kernel(mutated, causal), args).fused is None


def _conv_kernel(helper):
    def conv(out: "Tensor[f32, N, F, HO, WO]", x: "Tensor[f32, N, C, H, W]", w: "Tensor[f32, F, C, KH, KW]",
             bias: "Tensor[f32, F]", sh: SymbolDim, sw: SymbolDim, dh: SymbolDim, dw: SymbolDim, pt: SymbolDim,
             pb: SymbolDim, pl: SymbolDim, pr: SymbolDim, tf: SymbolDim, tc: SymbolDim, tn: SymbolDim,
             tho: SymbolDim, two: SymbolDim) -> None:
        helper(out, x, w, bias, sh, sw, dh, dw, pt, pb, pl, pr, tf, tc, tn, tho, two)

    return conv


@pytest.mark.parametrize(
    "old,new",
    [
        ("ph=row_lo - top,", "ph=row_lo - top + 1,"),
        ("taps = load(weight, [f0, ch, 0, 0]", "taps = load(weight, [f0, 0, 0, 0]"),
        ("window = load(image, [img, ch, row_lo, col_lo]", "window = load(image, [n0, ch, row_lo, col_lo]"),
        ("kernel.add(acc, acc, part)", "kernel.sub(acc, acc, part)"),
        ("sh=stride_h, sw=stride_w", "sh=stride_w, sw=stride_h"),
        ("pl=col_lo - left,", "pl=col_lo - left + 1,"),
        ("for img in loop(n0, min(n0 + tile_n, batch), 1):", "for img in loop(n0, min(n0 + tile_n, batch) - 1, 1):"),
        ("store(out, reshape(acc, [1, nf, rows, cols]), [img, f0, r0, c0]",
         "store(out, reshape(acc, [1, nf, rows, cols]), [img, f0, c0, r0]"),
    ],
)
def test_conv_mutations_do_not_fuse(old, new):
    x = np.zeros((1, 2, 9, 9), np.float32)
    w = np.zeros((2, 2, 3, 3), np.float32)
    args = (x, x, w, None, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 1, 3, 3)
    assert lowered(_conv_kernel(tiled_conv2d), args).fused is not None
    assert lowered(_conv_kernel(_mutate_source(tiled_conv2d, old, new)), args).fused is None


def _matmul_kernel(helper):
    def mm(out: "Tensor[f32, M, N]", lhs: "Tensor[f32, M, K]", rhs: "Tensor[f32, K, N]", bias: "Tensor[f32, N]",
           bm: SymbolDim, bn: SymbolDim, bk: SymbolDim) -> None:
        helper(out, lhs, rhs, bias, bm, bn, bk)

    return mm


@pytest.mark.parametrize(
    "old,new",
    [
        ("b_panel = load(rhs, [kk, col0]", "b_panel = load(rhs, [kk, 0]"),
        ("a_panel = load(lhs, [row0, kk]", "a_panel = load(lhs, [row0, 0]"),
        ("span = min(block_k, depth - kk)", "span = min(block_k, depth - kk - 1)"),
        ("bias_row = load(bias, [col0]", "bias_row = load(bias, [row0]"),
        ("fill(block, 0)", "fill(block, 1)"),
        ("store(out, block, [row0, col0]", "store(out, block, [col0, row0]"),
    ],
)
def test_matmul_mutations_do_not_fuse(old, new):
    a = np.zeros((16, 16), np.float32)
    args = (a, a, a, a[0], 4, 4, 4)
    assert lowered(_matmul_kernel(tiled_matmul), args).fused is not None
    assert lowered(_matmul_kernel(_mutate_source(tiled_matmul, old, new)), args).fused is None


def wrong_column_panel(out: "Tensor[f32, M, N]", lhs: "Tensor[f32, M, K]", rhs: "Tensor[f32, K, N]") -> None:
    # constant tiles of 72 x 80 x 48: the rhs panel ignores the column tile (offset 0 instead
    # of n0), which only shows when the column loop is sampled past its first trip
    m_size, k_size = lhs.get_shape()
    n_size = rhs.get_shape()[1]
    for m0 in loop(0, m_size, 72):
        for n0 in loop(0, n_size, 80):
            cm = min(72, m_size - m0)
            cn = min(80, n_size - n0)
            acc = alloc([cm, cn], NumericType.Float32, MemorySpace.TSM)
            fill(acc, 0)
            for k0 in loop(0, k_size, 48):
                ck = min(48, k_size - k0)
                lt = alloc([cm, ck], NumericType.Float32, MemorySpace.TSM)
                rt = alloc([ck, cn], NumericType.Float32, MemorySpace.TSM)
                deslice(lt, view(lhs, [m0, k0], [cm, ck], [1, 1]), [0, 0], [cm, ck], [1, 1])
                deslice(rt, view(rhs, [k0, 0], [ck, cn], [1, 1]), [0, 0], [ck, cn], [1, 1])
                part = alloc([cm, cn], NumericType.Float32, MemorySpace.TSM)
                kernel.matmul(part, lt, rt)
                kernel.add(acc, acc, part)
            deslice(out, acc, [m0, n0], [cm, cn], [1, 1])


def test_wrong_offset_with_large_constant_tiles_does_not_fuse():
    a = np.zeros((8, 8), np.float32)
    assert lowered(wrong_column_panel, (a, a, a)).fused is None
    # the same program with the right offset fuses
    right = _mutate_source(wrong_column_panel, "view(rhs, [k0, 0]", "view(rhs, [k0, n0]")
    assert lowered(right, (a, a, a)).fused is not None


def test_matching_samples_every_loop_past_its_first_trip():
    from kernelcode_generate_amd.passes import fuse

    a = np.zeros((8, 8), np.float32)
    func = mlir_gen(mm_static.matmul_inputs_static_tile_static_kernel, (a, a, a, None))
    kernel_aggregate(func)
    m = fuse._Match(fuse._Tracer(func))
    list(m.space.points(40))
    loops = fuse._all_loops(func)
    assert len(loops) == 3 and all(l.attrs["step"].is_const for l in loops)
    assert m.space.exercised(loops)
    assert all(m.space.max_trips[l.attrs["iv"]] >= 3 for l in loops)


def test_causal_form_is_recognised_from_the_row_mask():
    x = np.zeros((1, 1, 16, 8), np.float32)
    fused = lowered(flash_attention_scaled_causal_kernel, (x, x, x, x, 4, 4, 0.5)).fused
    assert fused.trailing_ints[0].value == 1 and fused.floats[0].arg == "scale"
    plain = lowered(flash_attention_scaled_kernel, (x, x, x, x, 4, 4, 0.5)).fused
    assert plain.trailing_ints[0].value == 0
    # a row mask that keeps one key too many is not causal attention
    wrong = _mutate_source(online_softmax_attention, "q0 + r + 1 - k0", "q0 + r + 2 - k0")
    assert lowered(_attention_kernel(wrong, True), (x, x, x, x, 4, 4, 0.5)).fused is None


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
    for name in ("symbol.for", "dma.alloc", "dma.fill", "dma.view", "dma.load", "dma.store", "dma.free",
                 "dma.reshape", "dma.transpose", "dma.broadcast", "kernel.matmul", "kernel.reduce", "kernel.exp",
                 "kernel.binary_elewise"):
        assert name in text
    assert "present(" not in text and "scale" in text


def test_pattern_fuse_entry_point():
    a = np.zeros((8, 8), np.float32)
    func = mlir_gen(my_gemm, (a, a, a, None, 4, 4, 4))
    assert pattern_fuse(func) is None  # before kernel-aggregate the K loop adds rounded partial products
    kernel_aggregate(func)
    assert pattern_fuse(func).family == "matmul"
    # the demo program accumulates in K order already
    demo = mlir_gen(matmul_inputs_dynamic_tile_dynamic_kernel, (a, a, a, None, 4, 4, 4))
    assert pattern_fuse(demo).family == "matmul"
