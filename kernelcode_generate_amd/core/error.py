"""Error taxonomy of the host-side mirror (kernel_gen/core/error.py:55-101 in the reference):
one exception type carrying a kind, a source module and, for execute-engine errors, the
stable failure phrase callers match on."""

from __future__ import annotations

from enum import Enum


class ErrorModule(str, Enum):
    GEN_KERNEL = "gen_kernel"
    PIPELINE = "pipeline"
    TARGET = "target"
    TOOLS = "tools"
    EXECUTE_ENGINE = "execute_engine"
    KERNEL = "kernel"


class ErrorKind(str, Enum):
    INVALID_VALUE = "invalid_value"
    CONTRACT = "contract"
    UNSUPPORTED = "unsupported"
    INTERNAL = "internal"


class KernelCodeError(Exception):
    """Project error: ``failure_phrase`` is set for execute-engine failures."""

    def __init__(self, kind: ErrorKind, module: ErrorModule, message: str, failure_phrase: str | None = None) -> None:
        super().__init__(message)
        self.kind = kind
        self.module = module
        self.failure_phrase = failure_phrase
