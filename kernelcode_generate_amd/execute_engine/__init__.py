"""gfx950 execute engine: the reference's compile/execute contract
(kernel_gen/execute_engine/__init__.py) with a registered ``gfx950`` compile strategy."""

from .compiler import (
    KNOWN_ERROR_PHRASES,
    CompiledKernel,
    CompileRequest,
    ExecuteRequest,
    ExecuteResult,
    ExecutionEngine,
)
from .gfx950_strategy import Gfx950CompileStrategy, register_gfx950_strategy
from .strategy import CompileStrategy, get_compile_strategy, register_compile_strategy

register_gfx950_strategy(override=True)

__all__ = [
    "KNOWN_ERROR_PHRASES",
    "CompileRequest",
    "CompileStrategy",
    "CompiledKernel",
    "ExecuteRequest",
    "ExecuteResult",
    "ExecutionEngine",
    "Gfx950CompileStrategy",
    "get_compile_strategy",
    "register_compile_strategy",
]
