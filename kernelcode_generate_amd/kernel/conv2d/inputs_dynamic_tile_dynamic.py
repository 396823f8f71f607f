"""Conv2d demo, runtime geometry and runtime tiles (the reference's
kernel/conv2d/inputs_dynamic_tile_dynamic.py:102-205): `tiled_conv2d` with stride,
dilation, the four pads and the five tile sizes as INT parameters."""

from __future__ import annotations

from kernelcode_generate_amd.kernel.conv2d.tiled import tiled_conv2d
from kernelcode_generate_amd.symbol_variable import SymbolDim


def conv2d_inputs_dynamic_tile_dynamic_kernel(
    out: "Tensor[f32, N, F, HO, WO]",
    input_tensor: "Tensor[f32, N, C, H, W]",
    weight: "Tensor[f32, F, C, KH, KW]",
    bias: "Tensor[f32, F]",
    stride_h: SymbolDim,
    stride_w: SymbolDim,
    dilation_h: SymbolDim,
    dilation_w: SymbolDim,
    pad_top: SymbolDim,
    pad_bottom: SymbolDim,
    pad_left: SymbolDim,
    pad_right: SymbolDim,
    tile_f: SymbolDim,
    tile_c: SymbolDim,
    tile_n: SymbolDim,
    tile_ho: SymbolDim,
    tile_wo: SymbolDim,
) -> None:
    tiled_conv2d(out, input_tensor, weight, bias, stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_bottom,
                 pad_left, pad_right, tile_f, tile_c, tile_n, tile_ho, tile_wo)
