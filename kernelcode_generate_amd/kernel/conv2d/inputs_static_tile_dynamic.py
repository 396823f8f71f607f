"""kernel/conv2d/inputs_static_tile_dynamic.py:120: stride 8 and seeded pads baked in, tiles
at run time."""

from __future__ import annotations

import random

from .._dsl import not_callable

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


def conv2d_inputs_static_tile_dynamic_kernel(out, input_tensor, weight, bias, tile_f, tile_c, tile_n, tile_ho,
                                             tile_wo) -> None:
    raise not_callable("conv2d_inputs_static_tile_dynamic_kernel")
