"""The allocation-free entry of generated per-operation kernels (kg_execute_entry_noalloc,
include/gfx950/kg_generated.h), called through the C ABI of the generated library.

It must give exactly the bits of kg_execute_entry (same kernel; its workspace comes from a
fixed __device__ scratch instead of hipMallocAsync), on two calls in a row with the second
input smaller than the first (the scratch keeps the first call's contents), and reject a
kernel whose per-workgroup workspace exceeds the scratch before launching anything.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from kernelcode_generate_amd import native
from kernelcode_generate_amd.dsl import mlir_gen
from kernelcode_generate_amd.execute_engine import ExecutionEngine
from kernelcode_generate_amd.gen_kernel import gen_kernel
from kernelcode_generate_amd.kernel.flash_attention.scaled import flash_attention_scaled_causal_kernel
from kernelcode_generate_amd.operation import kernel as dsl_kernel
from kernelcode_generate_amd.operation.dma import alloc, broadcast, deslice, load, store, view
from kernelcode_generate_amd.operation.scf import loop
from kernelcode_generate_amd.pipeline import get_pipeline
from kernelcode_generate_amd.symbol_variable import MemorySpace, NumericType, SymbolDim

pytestmark = pytest.mark.gpu


def _compile_per_op(fn, args):
    lowered = get_pipeline("gfx950-lowering", {"fuse": "false"}).run(mlir_gen(fn, args))
    assert lowered.fused is None
    compiled = ExecutionEngine("gfx950").compile(source=gen_kernel(lowered), function=fn.__name__)
    lib = ctypes.CDLL(compiled.soname_path)
    entries = []
    for name in ("kg_execute_entry", "kg_execute_entry_noalloc"):
        f = getattr(lib, name)
        f.argtypes = [ctypes.POINTER(native.KgArgSlot), ctypes.c_ulonglong]
        f.restype = ctypes.c_int
        entries.append(f)
    return compiled, lib, entries


def _call(entry, args) -> int:
    slots, keep = native.marshal_slots(args)
    rc = int(entry(slots, len(args)))
    del keep
    return rc


def test_noalloc_matches_allocating_entry(device, oracle_mod):
    import torch

    rng = np.random.default_rng(31)
    first = (1, 2, 45, 12)
    compiled, lib, (alloc_entry, noalloc_entry) = _compile_per_op(
        flash_attention_scaled_causal_kernel, tuple(np.zeros(first, np.float32) for _ in range(4)) + (12, 5, 0.29))
    try:
        for shape in (first, (1, 1, 20, 12)):  # the second call is smaller
            q, k, v = (rng.standard_normal(shape, dtype=np.float32) for _ in range(3))
            qt, kt, vt = (torch.from_numpy(a).to(device) for a in (q, k, v))
            outs = []
            for entry in (alloc_entry, noalloc_entry):
                out = torch.full(shape, float("nan"), device=device)
                print(f"[no-alloc] {shape} {entry.__name__}", flush=True)
                rc = _call(entry, (out, qt, kt, vt, 12, 5, 0.29))
                assert rc == 0, native.last_error()
                outs.append(out.cpu().numpy())
            assert np.array_equal(outs[0], outs[1]), f"{shape}: no-alloc entry differs"
            ref = oracle_mod.flash_attention_demo(q, k, v, 12, 5, scale=0.29, causal=True)
            ulp = np.spacing(np.abs(ref).astype(np.float32))
            assert np.all(np.abs(outs[1] - ref) <= 2 * ulp)
    finally:
        compiled.close()


def wide_rows_kernel(out: "Tensor[f32, R, C]", x: "Tensor[f32, R, C]", tile_r: SymbolDim) -> None:
    rows, cols = x.get_shape()
    for r0 in loop(0, rows, tile_r):
        cur = min(tile_r, rows - r0)
        t = alloc([cur, cols], NumericType.Float32, MemorySpace.TSM)
        deslice(t, view(x, [r0, 0], [cur, cols], [1, 1]), [0, 0], [cur, cols], [1, 1])
        m = alloc([cur, 1], NumericType.Float32, MemorySpace.TSM)
        dsl_kernel.reduce(m, t, kind=dsl_kernel.KernelReduceKind.MAX, axis=1, keepdim=True)
        full = alloc([cur, cols], NumericType.Float32, MemorySpace.TSM)
        broadcast(full, m)
        dsl_kernel.sub(t, t, full)
        deslice(out, t, [r0, 0], [cur, cols], [1, 1])


def test_noalloc_rejects_oversized_workspace(device):
    import torch

    x = torch.randn(2048, 4096, device=device)
    out = torch.empty_like(x)
    compiled, lib, (alloc_entry, noalloc_entry) = _compile_per_op(wide_rows_kernel, (x, out, 2048))
    try:
        print("[no-alloc] 64 MiB per workgroup", flush=True)
        assert _call(noalloc_entry, (out, x, 2048)) == -3  # 2 x 32 MiB of tiles per workgroup
        assert "scratch" in native.last_error()
        # a tile that fits runs, and agrees with the allocating entry
        small = torch.empty_like(x)
        assert _call(noalloc_entry, (small, x, 64)) == 0, native.last_error()
        assert _call(alloc_entry, (out, x, 64)) == 0, native.last_error()
        assert torch.equal(out, small)
        ref = x - x.max(dim=1, keepdim=True).values
        assert torch.equal(out, ref)
    finally:
        compiled.close()


def fixed_tile_rows(out: "Tensor[f32, R, C]", x: "Tensor[f32, R, C]") -> None:
    # every allocation has a constant extent: the generated library's scratch is sized exactly
    rows, cols = x.get_shape()
    for r0 in loop(0, rows, 4):
        t = load(x, [r0, 0], [4, 8], space=MemorySpace.TSM)
        dsl_kernel.add(t, t, t)
        store(out, t, [r0, 0], [4, 8])


def test_noalloc_exactly_sized_scratch(device):
    """A kernel whose allocations all have constant extents gets a scratch of exactly the
    largest grid's workspace plus the error word (4 x 8 fp32 = one 256-byte slice per
    workgroup, 2048 workgroups: 524,544 bytes, not the 32 MiB cap); two calls in a row, the
    second smaller, match the allocating entry."""

    import torch

    from kernelcode_generate_amd.gen_kernel import per_op

    x = torch.randn(4096, 8, device=device)
    lowered = get_pipeline("gfx950-lowering", {"fuse": "false"}).run(mlir_gen(fixed_tile_rows, (x, x)))
    assert per_op._Emitter(lowered.func).scratch_bytes() == 256 * per_op.MAX_GRID + 256
    compiled, lib, (alloc_entry, noalloc_entry) = _compile_per_op(fixed_tile_rows, (x, x))
    try:
        for rows in (4096, 64):  # 1024 workgroups, then 16
            xi = torch.randn(rows, 8, device=device)
            want, got = torch.full_like(xi, float("nan")), torch.full_like(xi, float("nan"))
            print(f"[no-alloc] exact scratch rows={rows}", flush=True)
            assert _call(alloc_entry, (want, xi)) == 0, native.last_error()
            assert _call(noalloc_entry, (got, xi)) == 0, native.last_error()
            assert torch.equal(got, want) and torch.equal(want, xi + xi)
    finally:
        compiled.close()
