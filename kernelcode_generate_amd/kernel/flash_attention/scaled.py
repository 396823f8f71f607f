"""Flash-attention variants the BASELINE configs need and the reference demos lack: a
softmax scale (kernel.mul of the score tile by a tile filled with `scale`) and, for the
causal kernel, the key bound min(seq_len, m0 + br) with a 0/-inf lower-triangular mask on
the diagonal tile. Expressible with the reference's existing DSL operations."""

from __future__ import annotations

from .._dsl import not_callable


def flash_attention_scaled_kernel(out, q, k, v, br, bc, scale) -> None:
    raise not_callable("flash_attention_scaled_kernel")


def flash_attention_scaled_causal_kernel(out, q, k, v, br, bc, scale) -> None:
    raise not_callable("flash_attention_scaled_causal_kernel")
