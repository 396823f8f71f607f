"""`dma` operations of the DSL (kernel_gen/operation/dma.py: alloc :134, fill :275,
broadcast :833, slice :945, deslice :978, view :1002, reshape :1046)."""

from __future__ import annotations

from ._marker import dsl_op

alloc = dsl_op("dma.alloc")          # alloc(shape, dtype, space) -> tile
fill = dsl_op("dma.fill")            # fill(target, value)          value: number, "inf", "-inf" or a float arg
view = dsl_op("dma.view")            # view(source, offsets, sizes, strides) -> view
reshape = dsl_op("dma.reshape")      # reshape(source, shape) -> view
slice = dsl_op("dma.slice")  # noqa: A001 - slice(source, offsets, sizes, strides, space) -> new tile
deslice = dsl_op("dma.deslice")      # deslice(target, source, offsets, sizes, strides)
broadcast = dsl_op("dma.broadcast")  # broadcast(target, source)

__all__ = ["alloc", "broadcast", "deslice", "fill", "reshape", "slice", "view"]
