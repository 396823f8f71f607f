"""Matmul demo, runtime shapes and tiles (the reference's
kernel/matmul/inputs_dynamic_tile_dynamic.py:57-113): `tiled_matmul` with the tile sizes as
INT parameters."""

from __future__ import annotations

from kernelcode_generate_amd.kernel.matmul.tiled import tiled_matmul
from kernelcode_generate_amd.symbol_variable import SymbolDim


def matmul_inputs_dynamic_tile_dynamic_kernel(
    out: "Tensor[f32, H, W]",
    lhs: "Tensor[f32, H, K]",
    rhs: "Tensor[f32, K, W]",
    bias: "Tensor[f32, W]",
    tile_h: SymbolDim,
    tile_w: SymbolDim,
    tile_k: SymbolDim,
) -> None:
    tiled_matmul(out, lhs, rhs, bias, tile_h, tile_w, tile_k)
