"""Compile-strategy registry (kernel_gen/execute_engine/strategy.py:92-144): one strategy
per registered target; duplicate registration needs override=True; a target without a
strategy fails with the phrase ``target_header_mismatch`` (no fallback to another target)."""

from __future__ import annotations

from typing import TYPE_CHECKING, Protocol, runtime_checkable

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..target import registry as target_registry

if TYPE_CHECKING:  # pragma: no cover
    from .compiler import CompiledKernel, CompileRequest


@runtime_checkable
class CompileStrategy(Protocol):
    def compile(self, request: "CompileRequest") -> "CompiledKernel":
        """Build a CompiledKernel or raise KernelCodeError with a failure phrase."""


_COMPILE_STRATEGIES: dict[str, CompileStrategy] = {}


def _error(phrase: str, detail: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.EXECUTE_ENGINE, f"{phrase}: {detail}", phrase)


def _validate_target(target: str) -> None:
    if not isinstance(target, str) or not target_registry._NAME_RE.match(target):
        raise _error("target_header_mismatch", f"invalid target name {target!r}")
    if not target_registry.is_registered(target):
        raise _error("target_header_mismatch", f"unregistered target {target!r}")


def register_compile_strategy(target: str, strategy: CompileStrategy, *, override: bool = False) -> None:
    _validate_target(target)
    if not isinstance(strategy, CompileStrategy):
        raise _error("compile_failed", "compile strategy must define compile")
    if target in _COMPILE_STRATEGIES and not override:
        raise _error("compile_failed", f"duplicate compile strategy: {target}")
    _COMPILE_STRATEGIES[target] = strategy


def get_compile_strategy(target: str) -> CompileStrategy:
    _validate_target(target)
    strategy = _COMPILE_STRATEGIES.get(target)
    if strategy is None:
        raise _error("target_header_mismatch", f"missing compile strategy: {target}")
    return strategy


def unregister_compile_strategy(target: str) -> None:
    _COMPILE_STRATEGIES.pop(target, None)
