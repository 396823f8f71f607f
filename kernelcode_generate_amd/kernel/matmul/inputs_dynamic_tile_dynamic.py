"""kernel/matmul/inputs_dynamic_tile_dynamic.py:57-113: symbolic shapes, runtime tiles."""

from __future__ import annotations

from .._dsl import not_callable


def matmul_inputs_dynamic_tile_dynamic_kernel(out, lhs, rhs, bias, tile_h, tile_w, tile_k) -> None:
    raise not_callable("matmul_inputs_dynamic_tile_dynamic_kernel")
