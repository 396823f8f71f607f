"""Drop-in check on the reference's own demo programs.

Each of the nine kernel functions of the reference's kernel/{matmul,conv2d,flash_attention}/
inputs_*.py is read as text -- never imported or executed -- and walked by this package's
front end (dsl.mlir_gen_source), its `from kernel_gen... import` names resolved to this
package's operations (dsl.source_namespace) and the module-level values its body reads
taken from the table below. Lowered by gfx950-lowering, each must fuse onto the expected
hand-written kernel with the expected operands (family, stride 8 and the seeded pads of the
static conv demos, the tile sizes); run operation by operation on the CPU (the numpy
interpreter of the per-operation semantics) each must reproduce the oracle's restatement of
the reference's loop nest bit for bit.

The reference checkout exists only where the tests are developed: elsewhere (the GPU box)
this module is skipped.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from kernelcode_generate_amd.dsl import mlir_gen_source
from kernelcode_generate_amd.pipeline import get_pipeline
from tests import ir_interp

REFERENCE_KERNELS = Path("/root/reference/kernel")
pytestmark = pytest.mark.skipif(not REFERENCE_KERNELS.is_dir(), reason="the reference checkout is not on this machine")

# The module-level values the static demos' kernel bodies read: the draws of the reference
# demos' seeded expressions (this package's demo modules draw them with the same seeds:
# test_constant_table_matches_the_seeded_demo_constants).
CONSTANTS = {
    "matmul/inputs_static_tile_static.py": {"_TILE_M": 48, "_TILE_N": 80, "_TILE_K": 56},
    "conv2d/inputs_static_tile_static.py": {
        "_STATIC_DILATION_H": 1, "_STATIC_DILATION_W": 1, "_STATIC_PAD_TOP": 3, "_STATIC_PAD_BOTTOM": 3,
        "_STATIC_PAD_LEFT": 4, "_STATIC_PAD_RIGHT": 0, "_STATIC_TILE_F": 7, "_STATIC_TILE_C": 18,
        "_STATIC_TILE_N": 3, "_STATIC_TILE_HO": 9, "_STATIC_TILE_WO": 8},
    "conv2d/inputs_static_tile_dynamic.py": {
        "_STATIC_DILATION_H": 1, "_STATIC_DILATION_W": 1, "_STATIC_PAD_TOP": 4, "_STATIC_PAD_BOTTOM": 3,
        "_STATIC_PAD_LEFT": 4, "_STATIC_PAD_RIGHT": 3},
    "flash_attention/inputs_static_tile_static.py": {"_STATIC_BR": 64, "_STATIC_BC": 80},
}

MATMUL = ("matmul/inputs_static_tile_static.py", "matmul/inputs_static_tile_dynamic.py",
          "matmul/inputs_dynamic_tile_dynamic.py")
CONV = ("conv2d/inputs_static_tile_static.py", "conv2d/inputs_static_tile_dynamic.py",
        "conv2d/inputs_dynamic_tile_dynamic.py")
ATTENTION = ("flash_attention/inputs_static_tile_static.py", "flash_attention/inputs_static_tile_dynamic.py",
             "flash_attention/inputs_dynamic_tile_dynamic.py")


def _function(path: str) -> str:
    family = path.split("/")[0]
    return f"{family}_{Path(path).stem}_kernel"


def _lower(path: str, args, fuse: bool = True):
    source = (REFERENCE_KERNELS / path).read_text()
    func = mlir_gen_source(source, _function(path), args, CONSTANTS.get(path))
    return get_pipeline("gfx950-lowering", {"fuse": fuse}).run(func)


def _value(sym, func, args) -> int:
    """A FusedCall operand at the runtime arguments `args`."""

    values = {p.name: a for p, a in zip(func.params, args)}

    def leaf(s):
        if s.op == "arg":
            return int(values[s.args[0]])
        if s.op == "dim":
            return int(values[s.args[0]].shape[s.args[1]])
        raise KeyError(s)

    return sym.evaluate(leaf)


def test_constant_table_matches_the_seeded_demo_constants():
    import importlib

    for path, table in CONSTANTS.items():
        module = importlib.import_module("kernelcode_generate_amd.kernel." + path[:-3].replace("/", "."))
        for name, value in table.items():
            assert getattr(module, name) == value, (path, name)


@pytest.mark.parametrize("path", MATMUL)
@pytest.mark.parametrize("with_bias", [False, True])
def test_reference_matmul_demo_fuses_and_runs(oracle_mod, path, with_bias):
    rng = np.random.default_rng(31)
    m, k, n = 97, 130, 75
    lhs = rng.standard_normal((m, k), dtype=np.float32)
    rhs = rng.standard_normal((k, n), dtype=np.float32)
    bias = rng.standard_normal(n, dtype=np.float32) if with_bias else None
    tiles = (48, 80, 56) if "static_tile_static" in path else (32, 24, 40)
    extra = () if "static_tile_static" in path else tiles
    args = (np.zeros((m, n), np.float32), lhs, rhs, bias, *extra)
    lw = _lower(path, args)
    assert lw.fused is not None and lw.fused.family == "matmul"
    assert lw.fused.memory == ("out", "lhs", "rhs", "bias")
    assert tuple(_value(s, lw.func, args) for s in lw.fused.ints) == tiles
    out = args[0]
    ir_interp.run(_lower(path, args, fuse=False).func, args)
    assert np.array_equal(out, oracle_mod.matmul_demo(lhs, rhs, bias, tiles))


@pytest.mark.parametrize("path", CONV)
def test_reference_conv_demo_fuses_and_runs(oracle_mod, path):
    rng = np.random.default_rng(37)
    if "static_tile_static" in path:
        geometry = ((8, 8), (1, 1), (3, 3, 4, 0))
        tiles, extra = (7, 18, 3, 9, 8), ()
        xs, ws = (2, 5, 37, 29), (6, 5, 3, 5)
    elif "static_tile_dynamic" in path:
        geometry = ((8, 8), (1, 1), (4, 3, 4, 3))
        tiles = (2, 3, 2, 2, 3)
        extra = tiles
        xs, ws = (3, 4, 30, 41), (5, 4, 3, 3)
    else:
        geometry = ((2, 1), (1, 2), (1, 2, 0, 3))
        tiles = (3, 2, 1, 4, 5)
        extra = geometry[0] + geometry[1] + geometry[2] + tiles
        xs, ws = (2, 3, 11, 13), (4, 3, 3, 2)
    stride, dil, pads = geometry
    x = rng.standard_normal(xs, dtype=np.float32)
    w = rng.standard_normal(ws, dtype=np.float32)
    b = rng.standard_normal(ws[0], dtype=np.float32)
    ho, wo = oracle_mod.conv2d_out_hw(xs[2], xs[3], ws[2], ws[3], stride, dil, pads)
    for bias in (None, b):
        out = np.zeros((xs[0], ws[0], ho, wo), np.float32)
        args = (out, x, w, bias, *extra)
        lw = _lower(path, args)
        assert lw.fused is not None and lw.fused.family == "conv2d"
        assert lw.fused.memory == ("out", "input_tensor", "weight", "bias")
        got = [_value(s, lw.func, args) for s in lw.fused.ints]
        assert got[:4] == [*stride, *dil] and (got[4], got[6]) == (pads[0], pads[2])
        # bottom / right: the least pads that give the same output extents
        assert oracle_mod.conv2d_out_hw(xs[2], xs[3], ws[2], ws[3], stride, dil, tuple(got[4:])) == (ho, wo)
        assert got[5] <= pads[1] and got[7] <= pads[3]
        ir_interp.run(_lower(path, args, fuse=False).func, args)
        assert np.array_equal(out, oracle_mod.conv2d_demo(x, w, bias, stride, dil, pads, tiles))


@pytest.mark.parametrize("path", ATTENTION)
def test_reference_attention_demo_fuses_and_runs(oracle_mod, path):
    rng = np.random.default_rng(41)
    shape = (1, 2, 45, 12)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
    tiles = (64, 80) if "static_tile_static" in path else (16, 10)
    extra = () if "static_tile_static" in path else tiles
    out = np.zeros(shape, np.float32)
    args = (out, q, k, v, *extra)
    lw = _lower(path, args)
    assert lw.fused is not None and lw.fused.family == "flash_attention"
    assert lw.fused.memory == ("out", "q", "k", "v")
    assert tuple(_value(s, lw.func, args) for s in lw.fused.ints) == tiles
    assert lw.fused.floats[0].value == 1.0 and lw.fused.trailing_ints[0].value == 0  # no scale, no mask
    ir_interp.run(_lower(path, args, fuse=False).func, args)
    assert np.array_equal(out, oracle_mod.flash_attention_demo(q, k, v, *tiles))


def test_reference_text_is_walked_not_run():
    """The front end never executes the demo module: its imports of the reference's own
    runtime (kernel.runner, kernel_gen.execute_engine, numpy) are not resolved at all."""

    source = (REFERENCE_KERNELS / MATMUL[1]).read_text()
    from kernelcode_generate_amd.dsl import source_namespace

    namespace = source_namespace(source)
    assert "run_lowering_demo" not in namespace and "ExecutionEngine" not in namespace and "np" not in namespace
    assert {"alloc", "fill", "view", "deslice", "loop", "kernel", "NumericType", "MemorySpace"} <= set(namespace)
    assert all(getattr(v, "dsl_op_name", None) or isinstance(v, type) or type(v).__name__ == "module"
               for v in namespace.values())
