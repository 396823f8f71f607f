"""Flash-attention demo, runtime tiles (the reference's
kernel/flash_attention/inputs_static_tile_dynamic.py:96): `online_softmax_attention` with
the query and key block sizes as INT parameters, no scale and no mask."""

from __future__ import annotations

from kernelcode_generate_amd.kernel.flash_attention.tiled import online_softmax_attention
from kernelcode_generate_amd.symbol_variable import SymbolDim


def flash_attention_inputs_static_tile_dynamic_kernel(
    out: "Tensor[f32, B, H, SL, D]",
    q: "Tensor[f32, B, H, SL, D]",
    k: "Tensor[f32, B, H, SL, D]",
    v: "Tensor[f32, B, H, SL, D]",
    br: SymbolDim,
    bc: SymbolDim,
) -> None:
    online_softmax_attention(out, q, k, v, br, bc, None, False)
