"""`nn` operations of the DSL used by the demos (kernel_gen/operation/nn/transpose.py:95)."""

from __future__ import annotations

from ._marker import dsl_op

transpose = dsl_op("nn.transpose")   # transpose(source, perm) -> new tile

__all__ = ["transpose"]
