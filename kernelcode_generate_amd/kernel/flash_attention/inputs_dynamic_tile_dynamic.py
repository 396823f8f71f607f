"""kernel/flash_attention/inputs_dynamic_tile_dynamic.py:96-195: symbolic shapes, runtime tiles."""

from __future__ import annotations

from .._dsl import not_callable


def flash_attention_inputs_dynamic_tile_dynamic_kernel(out, q, k, v, br, bc) -> None:
    raise not_callable("flash_attention_inputs_dynamic_tile_dynamic_kernel")
