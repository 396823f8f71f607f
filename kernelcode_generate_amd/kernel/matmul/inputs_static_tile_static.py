"""kernel/matmul/inputs_static_tile_static.py:56-110: out = lhs @ rhs (+ bias[None, :]) with
module-constant tiles (M, N, K loops; K-loop accumulation; rank-1 bias after the K loop)."""

from __future__ import annotations

import random

from .._dsl import not_callable

_STATIC_SHAPE_SEED = 2026051601
_STATIC_SHAPE_RNG = random.Random(_STATIC_SHAPE_SEED)
_STATIC_M = _STATIC_SHAPE_RNG.randint(160, 256)
_STATIC_K = _STATIC_SHAPE_RNG.randint(160, 256)
_STATIC_N = _STATIC_SHAPE_RNG.randint(160, 256)
_TILE_CANDIDATES = ((72, 56, 48), (48, 80, 56))
_TILE_M, _TILE_N, _TILE_K = random.Random(2026051700).choice(_TILE_CANDIDATES)


def matmul_inputs_static_tile_static_kernel(out, lhs, rhs, bias) -> None:
    raise not_callable("matmul_inputs_static_tile_static_kernel")
