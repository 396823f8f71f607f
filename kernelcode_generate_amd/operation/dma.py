"""`dma` operations of the DSL (kernel_gen/operation/dma.py: alloc :134, free :198,
fill :275, copy :722, broadcast :833, load :856, store :894, slice :945, deslice :978,
view :1002, reshape :1046, flatten :1083, cast :1119)."""

from __future__ import annotations

from ._marker import dsl_op

alloc = dsl_op("dma.alloc")          # alloc(shape, dtype, space) -> tile
free = dsl_op("dma.free")            # free(tile): ends the tile's lifetime (no data effect)
fill = dsl_op("dma.fill")            # fill(target, value)          value: number, "inf", "-inf" or a float arg
view = dsl_op("dma.view")            # view(source, offsets, sizes, strides) -> view
reshape = dsl_op("dma.reshape")      # reshape(source, shape) -> view
flatten = dsl_op("dma.flatten")      # flatten(source) -> rank-1 view of a contiguous source
slice = dsl_op("dma.slice")  # noqa: A001 - slice(source, offsets, sizes, strides=None, space=None) -> new tile
deslice = dsl_op("dma.deslice")      # deslice(target, source, offsets, sizes, strides=None)
load = dsl_op("dma.load")            # load(source, offsets, sizes, strides=None, space=None) -> new tile
store = dsl_op("dma.store")          # store(target, source, offsets, sizes, strides=None)
copy = dsl_op("dma.copy")            # copy(source, space) -> new tile holding the whole source
cast = dsl_op("dma.cast")            # cast(source, dtype, memoryspace=None) -> new tile of another element type
broadcast = dsl_op("dma.broadcast")  # broadcast(target, source)

__all__ = ["alloc", "broadcast", "cast", "copy", "deslice", "fill", "flatten", "free", "load", "reshape", "slice",
           "store", "view"]
