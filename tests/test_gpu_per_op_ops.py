"""The DSL operations the per-operation path runs beyond the demos' set: dma.load /
store / copy / cast / free / flatten and the arch launch queries (the reference's
kernel_gen/operation/dma.py:198,722,856,894,1083,1119 and operation/arch.py:652-803; the
cuda_sm89 backend accepts them, kernel_gen/dsl/gen_kernel/emit/cuda_sm89/source_bundle.py:
99-151). Each kernel runs through dsl_run on the GPU (the per-operation path: none of
them is a fused family) and data movement and casts must be bit-exact against numpy
slicing and torch's round-to-nearest-even casts."""

from __future__ import annotations

import numpy as np
import pytest

from kernelcode_generate_amd.operation.arch import (barrier, get_block_id, get_block_num, get_subthread_id,
                                                    get_subthread_num, get_thread_id, get_thread_num)
from kernelcode_generate_amd.operation.dma import cast, copy, flatten, free, load, reshape, store
from kernelcode_generate_amd.operation.scf import loop
from kernelcode_generate_amd.symbol_variable import MemorySpace, NumericType, SymbolDim
from kernelcode_generate_amd.tools import dsl_run

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def gfx950_target():
    from kernelcode_generate_amd.core.config import restore_config, set_target, snapshot_config

    snap = snapshot_config()
    set_target("gfx950")
    yield
    restore_config(snap)


def strided_copy(out: "Tensor[f32, R, C]", x: "Tensor[f32, R, C2]", tile: SymbolDim) -> None:
    # out[r, c] = x[r, 2 c + 1], through a loaded tile, a copy of it and a flattened view
    rows, cols = out.get_shape()
    for r0 in loop(0, rows, tile):
        h = min(tile, rows - r0)
        t = load(x, [r0, 1], [h, cols], [1, 2], space=MemorySpace.TSM)
        u = copy(t, MemorySpace.TSM)
        flat = flatten(u)
        store(out, reshape(flat, [h, cols]), [r0, 0], [h, cols])
        free(t)
        free(u)


def cast_rows(out: "Tensor[f16, R, C]", x: "Tensor[f32, R, C]", tile: SymbolDim) -> None:
    rows, cols = x.get_shape()
    for r0 in loop(0, rows, tile):
        h = min(tile, rows - r0)
        t = load(x, [r0, 0], [h, cols], space=MemorySpace.TSM)
        store(out, cast(t, NumericType.Float16), [r0, 0], [h, cols])


def cast_rows_bf16(out: "Tensor[bf16, R, C]", x: "Tensor[f32, R, C]", tile: SymbolDim) -> None:
    rows, cols = x.get_shape()
    for r0 in loop(0, rows, tile):
        h = min(tile, rows - r0)
        t = load(x, [r0, 0], [h, cols], space=MemorySpace.TSM)
        store(out, cast(t, NumericType.BFloat16), [r0, 0], [h, cols])


def widen_rows(out: "Tensor[f32, R, C]", x: "Tensor[f16, R, C]", tile: SymbolDim) -> None:
    rows, cols = x.get_shape()
    for r0 in loop(0, rows, tile):
        h = min(tile, rows - r0)
        store(out, cast(load(x, [r0, 0], [h, cols]), NumericType.Float32), [r0, 0], [h, cols])


def block_strided_rows(out: "Tensor[f32, R, C]", x: "Tensor[f32, R, C]") -> None:
    # the kernel distributes rows over the launch's blocks itself (arch-parallelize leaves it)
    rows, cols = x.get_shape()
    for r in loop(get_block_id(), rows, get_block_num()):
        row = load(x, [r, get_thread_id()], [get_thread_num(), cols - get_subthread_id()])
        barrier(visibility=None, scope=None)
        store(out, row, [r, get_subthread_id()], [get_subthread_num(), cols])


def _run(fn, args):
    result = dsl_run(fn, args, "gfx950-lowering")
    assert result.execute_result.ok, result.execute_result
    assert result.fused is None  # the per-operation path
    return result


def test_load_copy_flatten_store_strided(device):
    import torch

    rng = np.random.default_rng(5)
    x = rng.standard_normal((37, 41), dtype=np.float32)
    out = torch.full((37, 20), float("nan"), device=device)
    print("[per-op] strided load / copy / flatten / store, 37x20", flush=True)
    _run(strided_copy, (out, torch.from_numpy(x).to(device), 8))
    assert np.array_equal(out.cpu().numpy(), x[:, 1::2])


@pytest.mark.parametrize("fn,dtype", [(cast_rows, "float16"), (cast_rows_bf16, "bfloat16")])
def test_cast_rounds_to_nearest_even(device, fn, dtype):
    import torch

    rng = np.random.default_rng(6)
    # values that exercise rounding: random, halfway cases, tiny, huge, signed zeros, inf, nan
    x = (rng.standard_normal((33, 50)) * np.exp2(rng.integers(-30, 30, (33, 50)))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 1e-8, 3.0e38, 1.0 + 2.0 ** -11,
                        1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], np.float32)
    x.reshape(-1)[:special.size] = special
    tdt = getattr(torch, dtype)
    out = torch.zeros((33, 50), dtype=tdt, device=device)
    print(f"[per-op] cast f32 -> {dtype}", flush=True)
    _run(fn, (out, torch.from_numpy(x).to(device), 7))
    want = torch.from_numpy(x).to(tdt)
    got = out.cpu()
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16), want[~nan].view(torch.int16))


def test_cast_widens_exactly(device):
    import torch

    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((19, 23)).astype(np.float32)).to(torch.float16)
    out = torch.full((19, 23), float("nan"), device=device)
    print("[per-op] cast f16 -> f32", flush=True)
    _run(widen_rows, (out, x.to(device), 4))
    assert torch.equal(out.cpu(), x.float())


def test_launch_queries_distribute_rows(device):
    import torch

    rng = np.random.default_rng(9)
    x = rng.standard_normal((600, 24), dtype=np.float32)  # more rows than blocks: each block takes several
    out = torch.full((600, 24), float("nan"), device=device)
    print("[per-op] block-strided rows through arch.get_block_id / get_block_num", flush=True)
    result = _run(block_strided_rows, (out, torch.from_numpy(x).to(device)))
    assert result.module.parallel == ()  # arch-parallelize leaves a kernel that distributes itself
    assert np.array_equal(out.cpu().numpy(), x)
