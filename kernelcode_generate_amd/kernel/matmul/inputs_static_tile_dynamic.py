"""kernel/matmul/inputs_static_tile_dynamic.py:64-120: tiles are runtime int arguments."""

from __future__ import annotations

from .._dsl import not_callable


def matmul_inputs_static_tile_dynamic_kernel(out, lhs, rhs, bias, tile_h, tile_w, tile_k) -> None:
    raise not_callable("matmul_inputs_static_tile_dynamic_kernel")
