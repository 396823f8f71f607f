"""kernel/flash_attention/inputs_static_tile_static.py:90-190: softmax(Q K^T) V with Br/Bc
baked in (no scale, no mask)."""

from __future__ import annotations

import random

from .._dsl import not_callable

_STATIC_SHAPE_SEED = 2026052721
_STATIC_SHAPE_RNG = random.Random(_STATIC_SHAPE_SEED)
_STATIC_BATCH = _STATIC_SHAPE_RNG.choice((1, 2))
_STATIC_HEADS = _STATIC_SHAPE_RNG.choice((4, 8))
_STATIC_SEQ_LEN = _STATIC_SHAPE_RNG.choice((257, 321, 389))
_STATIC_DIM = _STATIC_SHAPE_RNG.choice((48, 64, 80))
_STATIC_TILE_CANDIDATES = ((48, 64), (64, 80), (80, 96))
_STATIC_BR, _STATIC_BC = random.Random(2026051727).choice(_STATIC_TILE_CANDIDATES)


def flash_attention_inputs_static_tile_static_kernel(out, q, k, v) -> None:
    raise not_callable("flash_attention_inputs_static_tile_static_kernel")
