"""Conv2d demo, static geometry and runtime tiles (the reference's
kernel/conv2d/inputs_static_tile_dynamic.py:120): `tiled_conv2d` with the seeded geometry
and the five tile sizes as INT parameters."""

from __future__ import annotations

import random

from kernelcode_generate_amd.kernel.conv2d.tiled import tiled_conv2d
from kernelcode_generate_amd.symbol_variable import SymbolDim

_STATIC_SHAPE_SEED = 2026052702
_STATIC_SHAPE_RNG = random.Random(_STATIC_SHAPE_SEED)
_STATIC_BATCH = _STATIC_SHAPE_RNG.randint(4, 6)
_STATIC_IN_CHANNELS = _STATIC_SHAPE_RNG.randint(48, 64)
_STATIC_INPUT_H = _STATIC_SHAPE_RNG.randint(241, 289)
_STATIC_INPUT_W = _STATIC_SHAPE_RNG.randint(225, 273)
_STATIC_OUT_CHANNELS = _STATIC_SHAPE_RNG.randint(18, 24)
_STATIC_KERNEL_H = _STATIC_SHAPE_RNG.choice((3, 5))
_STATIC_KERNEL_W = _STATIC_SHAPE_RNG.choice((3, 5))
_STATIC_STRIDE_H = 8
_STATIC_STRIDE_W = 8
_STATIC_DILATION_H = 1
_STATIC_DILATION_W = 1
_STATIC_PAD_TOP = _STATIC_SHAPE_RNG.choice((0, 1, 2, 3, 4))
_STATIC_PAD_BOTTOM = _STATIC_SHAPE_RNG.choice((0, 1, 2, 3, 4))
_STATIC_PAD_LEFT = _STATIC_SHAPE_RNG.choice((0, 1, 2, 3, 4))
_STATIC_PAD_RIGHT = _STATIC_SHAPE_RNG.choice((0, 1, 2, 3, 4))


def conv2d_inputs_static_tile_dynamic_kernel(
    out: "Tensor[f32, N, F, HO, WO]",
    input_tensor: "Tensor[f32, N, C, H, W]",
    weight: "Tensor[f32, F, C, KH, KW]",
    bias: "Tensor[f32, F]",
    tile_f: SymbolDim,
    tile_c: SymbolDim,
    tile_n: SymbolDim,
    tile_ho: SymbolDim,
    tile_wo: SymbolDim,
) -> None:
    tiled_conv2d(out, input_tensor, weight, bias, _STATIC_STRIDE_H, _STATIC_STRIDE_W, _STATIC_DILATION_H,
                 _STATIC_DILATION_W, _STATIC_PAD_TOP, _STATIC_PAD_BOTTOM, _STATIC_PAD_LEFT, _STATIC_PAD_RIGHT,
                 tile_f, tile_c, tile_n, tile_ho, tile_wo)
