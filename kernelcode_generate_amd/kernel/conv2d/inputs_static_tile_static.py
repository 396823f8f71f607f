"""Conv2d demo, static geometry and static tiles (the reference's
kernel/conv2d/inputs_static_tile_static.py:115-215): `tiled_conv2d` with stride 8, the seeded
dilation and asymmetric pads, and the seeded tile sizes. The constants are drawn with the
reference demo's seeds, so the demo runs the same problem."""

from __future__ import annotations

import random

from kernelcode_generate_amd.kernel.conv2d.tiled import tiled_conv2d

_STATIC_SHAPE_SEED = 2026052701
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
_STATIC_TILE_CANDIDATES = ((8, 16, 4, 8, 9), (7, 18, 3, 9, 8), (6, 20, 2, 10, 7))
_STATIC_TILE_F, _STATIC_TILE_C, _STATIC_TILE_N, _STATIC_TILE_HO, _STATIC_TILE_WO = random.Random(2026051721).choice(
    _STATIC_TILE_CANDIDATES
)


def conv2d_inputs_static_tile_static_kernel(
    out: "Tensor[f32, N, F, HO, WO]",
    input_tensor: "Tensor[f32, N, C, H, W]",
    weight: "Tensor[f32, F, C, KH, KW]",
    bias: "Tensor[f32, F]",
) -> None:
    tiled_conv2d(out, input_tensor, weight, bias, _STATIC_STRIDE_H, _STATIC_STRIDE_W, _STATIC_DILATION_H,
                 _STATIC_DILATION_W, _STATIC_PAD_TOP, _STATIC_PAD_BOTTOM, _STATIC_PAD_LEFT, _STATIC_PAD_RIGHT,
                 _STATIC_TILE_F, _STATIC_TILE_C, _STATIC_TILE_N, _STATIC_TILE_HO, _STATIC_TILE_WO)
