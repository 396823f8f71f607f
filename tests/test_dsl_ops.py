"""CPU tests of the DSL operations beyond the demos' set (dma.load / store / copy / cast /
free / flatten, the arch launch queries and barrier): the front end's IR, executed by the
numpy interpreter of the per-operation semantics, reproduces numpy slicing and casting bit
for bit, and unsupported operations fail in the front end with an error naming them. The
same kernels run on the GPU in test_gpu_per_op_ops.py."""

from __future__ import annotations

import numpy as np
import pytest

from kernelcode_generate_amd.core.error import KernelCodeError
from kernelcode_generate_amd.dsl import mlir_gen
from kernelcode_generate_amd.gen_kernel.per_op import QUERY_GRID, parallel_loops, uses_block_queries
from kernelcode_generate_amd.ir import format_func
from kernelcode_generate_amd.operation.arch import get_dynamic_memory
from kernelcode_generate_amd.operation.dma import alloc, free
from kernelcode_generate_amd.passes import pattern_fuse
from kernelcode_generate_amd.symbol_variable import MemorySpace
from tests import ir_interp
from tests.test_gpu_per_op_ops import block_strided_rows, cast_rows, cast_rows_bf16, strided_copy, widen_rows


def test_strided_load_copy_flatten_store():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((37, 41), dtype=np.float32)
    out = np.full((37, 20), np.nan, np.float32)
    func = mlir_gen(strided_copy, (out, x, 8))
    text = format_func(func)
    for name in ("dma.load", "dma.copy", "dma.reshape", "dma.store", "dma.free"):
        assert name in text
    assert pattern_fuse(func) is None
    ir_interp.run(func, (out, x, 8))
    assert np.array_equal(out, x[:, 1::2])


def test_casts_round_to_nearest_even():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((33, 50)) * np.exp2(rng.integers(-30, 30, (33, 50)))).astype(np.float32)
    out = np.zeros((33, 50), np.float16)
    ir_interp.run(mlir_gen(cast_rows, (out, x, 7)), (out, x, 7))
    with np.errstate(over="ignore"):
        half = x.astype(np.float16)
    assert np.array_equal(out.view(np.int16), half.view(np.int16))
    # bf16 (kept as float32 here): the interpreter's rounding against a closed form of RNE
    out32 = np.zeros((33, 50), np.float32)
    func = mlir_gen(cast_rows_bf16, (out32, x, 7))
    ir_interp.run(func, (out32, x, 7))
    bits = x.view(np.uint32).astype(np.uint64)
    rne = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    assert np.array_equal(out32.view(np.uint32), rne.astype(np.uint32))
    wide = np.zeros((33, 50), np.float32)
    ir_interp.run(mlir_gen(widen_rows, (wide, half, 4)), (wide, half, 4))
    assert np.array_equal(wide, half.astype(np.float32))


def test_launch_queries_distribute_rows():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((600, 24), dtype=np.float32)
    out = np.full((600, 24), np.nan, np.float32)
    func = mlir_gen(block_strided_rows, (out, x))
    assert uses_block_queries(func) and parallel_loops(func) == []
    assert "arch.get_block_id()" in format_func(func) and "arch.barrier" in format_func(func)
    ir_interp.run(func, (out, x), blocks=QUERY_GRID)
    assert np.array_equal(out, x)


def test_unsupported_operations_are_named():
    def dynamic_memory(out: "Tensor[f32, N]") -> None:
        scratch = get_dynamic_memory(MemorySpace.TSM)  # noqa: F841

    def free_argument(out: "Tensor[f32, N]") -> None:
        free(out)

    def bad_cast(out: "Tensor[f32, N]") -> None:
        t = alloc([4], "f64", MemorySpace.TSM)  # noqa: F841

    a = np.zeros(4, np.float32)
    with pytest.raises(KernelCodeError, match="arch.get_dynamic_memory is not supported"):
        mlir_gen(dynamic_memory, (a,))
    with pytest.raises(KernelCodeError, match="dma.free"):
        mlir_gen(free_argument, (a,))
    with pytest.raises(KernelCodeError, match="element type"):
        mlir_gen(bad_cast, (a,))


def _lower_per_op(fn, args):
    from kernelcode_generate_amd.pipeline import get_pipeline

    return get_pipeline("gfx950-lowering", {"fuse": "false"}).run(mlir_gen(fn, args))


def test_noalloc_scratch_is_bounded_by_static_workspace():
    """The allocation-free entry's __device__ scratch: exact for kernels whose allocations all
    have constant extents, the 32 MiB cap otherwise (extents that depend on the arguments)."""

    from kernelcode_generate_amd.gen_kernel import per_op
    from tests.test_zz_no_alloc import fixed_tile_rows

    x = np.zeros((64, 8), np.float32)
    fixed = per_op._Emitter(_lower_per_op(fixed_tile_rows, (x, x)).func)
    assert fixed.scratch_bytes() == 256 * per_op.MAX_GRID + 256
    assert f"char scratch[{256 * per_op.MAX_GRID + 256}];" in fixed.source("fixed_tile_rows")
    dynamic = per_op._Emitter(_lower_per_op(cast_rows, (np.zeros((64, 8), np.float16), x, 4)).func)
    assert dynamic.scratch_bytes() == per_op.SCRATCH_BYTES == 32 << 20
