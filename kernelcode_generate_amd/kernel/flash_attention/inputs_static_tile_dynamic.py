"""kernel/flash_attention/inputs_static_tile_dynamic.py:96: Br/Bc at run time."""

from __future__ import annotations

from .._dsl import not_callable


def flash_attention_inputs_static_tile_dynamic_kernel(out, q, k, v, br, bc) -> None:
    raise not_callable("flash_attention_inputs_static_tile_dynamic_kernel")
