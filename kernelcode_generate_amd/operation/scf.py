"""`scf.loop` of the DSL (kernel_gen/operation/scf.py:336): `for i in loop(start, end, step)`
becomes a symbol.for over [start, end) with a positive step."""

from __future__ import annotations

from ._marker import dsl_op

loop = dsl_op("scf.loop")

__all__ = ["loop"]
