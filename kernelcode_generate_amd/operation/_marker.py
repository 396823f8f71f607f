"""DSL operations are markers: the front end (dsl.mlir_gen) reads a kernel's Python source
and maps each call to an IR operation; calling one directly is a usage error."""

from __future__ import annotations

from ..core.error import ErrorKind, ErrorModule, KernelCodeError


def dsl_op(name: str):
    def op(*args, **kwargs):
        raise KernelCodeError(ErrorKind.CONTRACT, ErrorModule.KERNEL,
                              f"{name} is a DSL operation: it runs inside a kernel passed to dsl_run(kernel, args, "
                              f"'gfx950-lowering'), not as a Python call")

    op.__name__ = name.split(".")[-1]
    op.__qualname__ = op.__name__
    op.dsl_op_name = name
    return op
