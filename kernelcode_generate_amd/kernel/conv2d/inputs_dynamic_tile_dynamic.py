"""kernel/conv2d/inputs_dynamic_tile_dynamic.py:102-205: symbolic shapes, runtime stride,
dilation, pads and tiles."""

from __future__ import annotations

from .._dsl import not_callable


def conv2d_inputs_dynamic_tile_dynamic_kernel(out, input_tensor, weight, bias, stride_h, stride_w, dilation_h,
                                              dilation_w, pad_top, pad_bottom, pad_left, pad_right, tile_f, tile_c,
                                              tile_n, tile_ho, tile_wo) -> None:
    raise not_callable("conv2d_inputs_dynamic_tile_dynamic_kernel")
