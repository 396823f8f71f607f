"""`kernel` operations of the DSL (kernel_gen/operation/kernel/__init__.py:1-40 of the
reference): out-first helpers on memory tiles."""

from __future__ import annotations

from enum import Enum

from ._marker import dsl_op


class KernelReduceKind(Enum):
    """kernel.reduce kinds (kernel_gen/operation/kernel/reduction.py:152)."""

    MAX = "max"
    SUM = "sum"


class KernelBinaryElewiseKind(Enum):
    """kernel.binary_elewise kinds (kernel_gen/dialect/kernel/operation/binary.py:221)."""

    ADD = "add"
    SUB = "sub"
    MUL = "mul"
    TRUEDIV = "truediv"
    MAX = "max"


matmul = dsl_op("kernel.matmul")              # matmul(out, lhs, rhs, *, acc=False)
img2col2d = dsl_op("kernel.img2col2d")        # img2col2d(out, input, kh=, kw=, sh=, sw=, dh=, dw=, ph=, pw=, pl=, pr=)
exp = dsl_op("kernel.exp")                    # exp(out, input)
reduce = dsl_op("kernel.reduce")              # reduce(out, input, kind=, axis=, keepdim=)
binary_elewise = dsl_op("kernel.binary_elewise")  # binary_elewise(out, lhs, rhs, kind=)
add = dsl_op("kernel.add")
sub = dsl_op("kernel.sub")
mul = dsl_op("kernel.mul")
truediv = dsl_op("kernel.truediv")
max = dsl_op("kernel.max")  # noqa: A001 - the DSL's name

__all__ = ["KernelBinaryElewiseKind", "KernelReduceKind", "add", "binary_elewise", "exp", "img2col2d", "matmul", "max",
           "mul", "reduce", "sub", "truediv"]
