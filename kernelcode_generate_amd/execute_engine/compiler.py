"""Execute-engine facade for the gfx950 target, with the reference's public contract
(kernel_gen/execute_engine/compiler.py:119-475):

- ``ExecutionEngine(target).compile(source, function) -> CompiledKernel`` through the
  strategy registered for the target;
- ``CompiledKernel.execute(args) -> ExecuteResult``: args in DSL parameter order, entry
  ``kg_execute_entry``, non-zero status -> ``KernelCodeError`` with failure phrase
  ``runtime_throw_or_abort`` (:348-352), unknown entry -> ``symbol_resolve_failed``;
- the stable failure phrases of :68-90.

Differences, all additive: execution is enabled for ``gfx950`` (the reference gates it to
cpu/npu_demo/cuda_sm89 at :292-296); ``ExecuteRequest.stream`` may name a HIP stream
(torch.cuda.Stream or raw handle), in which case the launch is only enqueued on it, while
``None`` keeps the reference's synchronous behaviour; ``ExecuteResult.elapsed_ms`` is the
GPU time of the call measured with HIP events (declared but never set in the reference,
:180, :353-359).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any, Callable

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from . import runtime_args as _runtime_args
from .strategy import get_compile_strategy

TARGET_HEADER_MISMATCH = "target_header_mismatch"
SOURCE_EMPTY_OR_INVALID = "source_empty_or_invalid"
COMPILE_FAILED = "compile_failed"
TEMPLATE_INSTANCE_REQUIRED = "template_instance_required"
SYMBOL_RESOLVE_FAILED = "symbol_resolve_failed"
RUNTIME_THROW_OR_ABORT = "runtime_throw_or_abort"
STREAM_NOT_SUPPORTED = "stream_not_supported"
FUNCTION_OUTPUT_CAPTURE_NOT_SUPPORTED = "function_output_capture_not_supported"
EXECUTION_UNSUPPORTED = "execution_unsupported"
KNOWN_ERROR_PHRASES = frozenset(
    {
        TARGET_HEADER_MISMATCH,
        SOURCE_EMPTY_OR_INVALID,
        COMPILE_FAILED,
        TEMPLATE_INSTANCE_REQUIRED,
        SYMBOL_RESOLVE_FAILED,
        RUNTIME_THROW_OR_ABORT,
        STREAM_NOT_SUPPORTED,
        FUNCTION_OUTPUT_CAPTURE_NOT_SUPPORTED,
        EXECUTION_UNSUPPORTED,
    }
)
EXECUTABLE_TARGETS = frozenset({"gfx950"})


def execute_engine_error(failure_phrase: str, detail: str = "") -> KernelCodeError:
    if failure_phrase not in KNOWN_ERROR_PHRASES:
        raise KernelCodeError(ErrorKind.CONTRACT, ErrorModule.EXECUTE_ENGINE, f"unknown failure phrase: {failure_phrase}")
    message = failure_phrase if not detail else f"{failure_phrase}: {detail}"
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.EXECUTE_ENGINE, message, failure_phrase)


@dataclass(frozen=True)
class CompileRequest:
    source: str
    target: str
    function: str
    entry_point: str = "kg_execute_entry"
    compiler: str | None = None
    compiler_flags: tuple[str, ...] = ("-std=c++17",)
    link_flags: tuple[str, ...] = ()


@dataclass(frozen=True)
class ExecuteRequest:
    args: tuple
    entry_point: str | None = None
    capture_function_output: bool = False
    stream: Any = None


@dataclass(frozen=True)
class ExecuteResult:
    ok: bool
    status_code: int
    failure_phrase: str | None
    compile_stdout: str = ""
    compile_stderr: str = ""
    run_stdout: str = ""
    run_stderr: str = ""
    elapsed_ms: float = 0.0


def _stream_handle(stream: Any) -> int:
    if isinstance(stream, int):
        return stream
    handle = getattr(stream, "cuda_stream", None)
    if handle is None:
        raise execute_engine_error(STREAM_NOT_SUPPORTED, "stream must be a torch.cuda.Stream or a hipStream_t handle")
    return int(handle)


@dataclass(frozen=True)
class CompiledKernel:
    target: str
    soname_path: str
    function: str
    entry_point: str
    compile_stdout: str = ""
    compile_stderr: str = ""
    allow_absent_memory_args: tuple[_runtime_args.AllowAbsentMemoryArg, ...] = field(default_factory=tuple, repr=False,
                                                                                     compare=False)
    _cleanup: Callable[[], None] | None = field(default=None, repr=False, compare=False)
    _state: dict = field(default_factory=dict, init=False, repr=False, compare=False)

    def close(self) -> None:
        cleanup = self._state.pop("cleanup", self._cleanup) if "closed" not in self._state else None
        self._state["closed"] = True
        self._state.pop("invoke", None)
        if cleanup is not None:
            cleanup()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def _invoker(self, entry_point: str):
        if self._state.get("closed"):
            raise execute_engine_error(SYMBOL_RESOLVE_FAILED, "compiled kernel is closed")
        invoke = self._state.get("invoke")
        if invoke is None:
            invoke = _runtime_args.load_entry_point(self.soname_path, entry_point)
            self._state["invoke"] = invoke
        return invoke

    def execute(self, args: tuple | None = None, *, request: ExecuteRequest | None = None, entry_point: str | None = None,
                capture_function_output: bool = False, stream: Any = None) -> ExecuteResult:
        if request is not None:
            args = request.args
            entry_point = request.entry_point if entry_point is None else entry_point
            capture_function_output = request.capture_function_output
            stream = request.stream
        if self.target not in EXECUTABLE_TARGETS:
            raise execute_engine_error(EXECUTION_UNSUPPORTED, "compiled target does not expose runtime execution")
        if args is None:
            raise execute_engine_error(RUNTIME_THROW_OR_ABORT, "args must be provided")
        if not isinstance(args, tuple):
            raise execute_engine_error(RUNTIME_THROW_OR_ABORT, "args must be a tuple")
        resolved = self.entry_point if entry_point is None else entry_point
        if not isinstance(resolved, str) or not resolved.strip():
            raise execute_engine_error(SYMBOL_RESOLVE_FAILED, "entry_point is empty")
        if resolved != self.entry_point:
            raise execute_engine_error(SYMBOL_RESOLVE_FAILED, "entry_point mismatch")
        if capture_function_output:
            raise execute_engine_error(FUNCTION_OUTPUT_CAPTURE_NOT_SUPPORTED,
                                       "function output capture is an npu_demo cost-summary feature")
        _runtime_args.validate_args(args, self.allow_absent_memory_args)
        invoke = self._invoker(resolved)

        import torch

        from .. import native

        if stream is None:
            # synchronous, like the reference; GPU time of the call from HIP events
            native.set_launch_mode(True, None)
            begin = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            null_stream = torch.cuda.default_stream()
            begin.record(null_stream)
            t0 = time.perf_counter()
            status = invoke(args)
            end.record(null_stream)
            end.synchronize()
            elapsed = begin.elapsed_time(end) if status == 0 else (time.perf_counter() - t0) * 1e3
        else:
            native.set_launch_mode(False, _stream_handle(stream))
            try:
                status = invoke(args)
            finally:
                native.set_launch_mode(True, None)
            elapsed = 0.0
        if status != 0:
            detail = native.last_error()
            raise execute_engine_error(RUNTIME_THROW_OR_ABORT, f"entry_point returned non-zero ({status}): {detail}")
        return ExecuteResult(ok=True, status_code=0, failure_phrase=None, compile_stdout=self.compile_stdout,
                             compile_stderr=self.compile_stderr, elapsed_ms=float(elapsed))


@dataclass(frozen=True)
class ExecutionEngine:
    target: str
    compiler: str | None = None
    compiler_flags: tuple[str, ...] = ("-std=c++17",)
    link_flags: tuple[str, ...] = ()

    def compile(self, source: str | None = None, function: str | None = None, *, request: CompileRequest | None = None,
                entry_point: str = "kg_execute_entry") -> CompiledKernel:
        if request is not None:
            if source is not None or function is not None:
                raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "request cannot be combined with source or function")
            compile_request = request
        else:
            compile_request = CompileRequest(source=source, target=self.target, function=function, entry_point=entry_point,
                                             compiler=self.compiler, compiler_flags=self.compiler_flags,
                                             link_flags=self.link_flags)
        if not isinstance(compile_request.source, str) or not compile_request.source.strip():
            raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "source must be a non-empty string")
        if not isinstance(compile_request.function, str) or not compile_request.function.strip():
            raise execute_engine_error(SOURCE_EMPTY_OR_INVALID, "function must be a non-empty string")
        strategy = get_compile_strategy(compile_request.target)
        return strategy.compile(compile_request)
