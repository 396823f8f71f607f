"""Shared helper: DSL kernel identities are run through dsl_run, never called directly."""

from __future__ import annotations

from ..core.error import ErrorKind, ErrorModule, KernelCodeError


def not_callable(name: str) -> KernelCodeError:
    return KernelCodeError(
        ErrorKind.CONTRACT,
        ErrorModule.KERNEL,
        f"{name} is a DSL kernel: run it with dsl_run({name}, args, 'gfx950-lowering') or run_gfx950_demo",
    )
