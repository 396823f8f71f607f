"""Runtime-argument classification and slot marshalling for compiled gfx950 kernels.

Mirrors kernel_gen/execute_engine/runtime_args.py: args are bound in DSL parameter order;
memory args (torch ROCm tensors) must be contiguous (:532-533); ``None`` is accepted only
at an index the source declares with ``// kg.allow_absent_memory_args: <idx>:<dtype>:<rank>``
(:497-516, builtin_strategy/common.py:496-532); Python ints / floats become INT / FLOAT
slots; the C slot is the reference's ``_CArgSlot`` (:217-237). dtype codes are the
reference's 1-4 plus 5 = float16 and 6 = bfloat16.
"""

from __future__ import annotations

import ctypes
import re
from dataclasses import dataclass
from numbers import Integral, Real
from typing import Any, Callable

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..native import DTYPE_CODES, KgArgSlot, marshal_slots

RUNTIME_THROW_OR_ABORT = "runtime_throw_or_abort"
SYMBOL_RESOLVE_FAILED = "symbol_resolve_failed"
_ALLOW_ABSENT_RE = re.compile(r"//\s*kg\.allow_absent_memory_args:\s*(?P<body>[^\n]*)")
_DTYPE_ALIASES = {
    "float": "float32", "f32": "float32", "float32": "float32",
    "double": "float64", "f64": "float64", "float64": "float64",
    "int": "int32", "i32": "int32", "int32": "int32",
    "i64": "int64", "int64": "int64", "longlong": "int64",
    "half": "float16", "f16": "float16", "float16": "float16",
    "bf16": "bfloat16", "bfloat16": "bfloat16",
}


@dataclass(frozen=True)
class AllowAbsentMemoryArg:
    index: int
    dtype: str
    rank: int


def runtime_error(phrase: str, detail: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.EXECUTE_ENGINE, f"{phrase}: {detail}", phrase)


def parse_allow_absent(source: str | None) -> tuple[AllowAbsentMemoryArg, ...]:
    """``// kg.allow_absent_memory_args: 3:float:1;...`` -> specs."""

    if not source:
        return ()
    specs: list[AllowAbsentMemoryArg] = []
    for match in _ALLOW_ABSENT_RE.finditer(source):
        for item in match.group("body").split(";"):
            item = item.strip()
            if not item:
                continue
            parts = item.split(":")
            if len(parts) != 3:
                raise runtime_error("source_empty_or_invalid", f"malformed allow_absent entry {item!r}")
            idx, dtype, rank = parts
            specs.append(AllowAbsentMemoryArg(int(idx), _DTYPE_ALIASES.get(dtype.strip(), dtype.strip()), int(rank)))
    return tuple(specs)


def _is_memory(value: Any) -> bool:
    return hasattr(value, "data_ptr") and hasattr(value, "shape") and hasattr(value, "stride")


def validate_args(args: tuple, allow_absent: tuple[AllowAbsentMemoryArg, ...]) -> None:
    absent = {spec.index for spec in allow_absent}
    for idx, arg in enumerate(args):
        if arg is None:
            if idx not in absent:
                raise runtime_error(RUNTIME_THROW_OR_ABORT,
                                    f"None runtime arg requires allow-absent memory metadata at position {idx}")
            continue
        if isinstance(arg, bool):
            raise runtime_error(RUNTIME_THROW_OR_ABORT, f"unsupported runtime arg at position {idx}")
        if isinstance(arg, (Integral, Real)):
            continue
        if not _is_memory(arg):
            raise runtime_error(RUNTIME_THROW_OR_ABORT, f"unsupported runtime arg at position {idx}")
        dtype = str(getattr(arg, "dtype", "")).replace("torch.", "")
        if dtype not in DTYPE_CODES:
            raise runtime_error(RUNTIME_THROW_OR_ABORT, f"unsupported memory dtype {dtype} at position {idx}")
        if hasattr(arg, "is_contiguous") and not arg.is_contiguous():
            raise runtime_error(RUNTIME_THROW_OR_ABORT, f"memory arg is not contiguous at position {idx}")
        if getattr(getattr(arg, "device", None), "type", "cuda") != "cuda":
            raise runtime_error(RUNTIME_THROW_OR_ABORT,
                                f"memory arg at position {idx} must live in device memory (ROCm tensor)")


def load_entry_point(soname_path: str, entry_point: str) -> Callable[[tuple], int]:
    try:
        library = ctypes.CDLL(soname_path)
    except OSError as exc:
        raise runtime_error(SYMBOL_RESOLVE_FAILED, f"unable to load shared object: {exc}") from exc
    try:
        symbol = getattr(library, entry_point)
    except AttributeError as exc:
        raise runtime_error(SYMBOL_RESOLVE_FAILED, f"entry_point '{entry_point}' is missing") from exc
    symbol.argtypes = [ctypes.POINTER(KgArgSlot), ctypes.c_ulonglong]
    symbol.restype = ctypes.c_int

    def invoke(args: tuple) -> int:
        array, keep = marshal_slots(args)
        status = int(symbol(array, ctypes.c_ulonglong(len(args))))
        del keep
        return status

    invoke.library = library  # keep the handle alive with the callable
    return invoke
