"""ctypes binding of libkg_gfx950.so, the gfx950 C ABI declared in include/kg_gfx950.h.

The slot structure is byte-for-byte the reference's ``_CArgSlot``
(kernel_gen/execute_engine/runtime_args.py:217-237) and the marshalling follows
``_RuntimeArgSupport.marshal_slots_for_abi`` (runtime_args.py:590-664): memory slots carry
a data pointer, element shape and element strides; ``None`` is an absent memory slot
(data = NULL, shape (0,), stride (1,)); Python ints and floats become INT / FLOAT slots.
Memory arguments must be ROCm device tensors: the library refuses host pointers.

There is no CPU fallback: if the shared object is missing this module raises.
"""

from __future__ import annotations

import ctypes
import os
from numbers import Integral, Real
from pathlib import Path
from typing import Any, Sequence

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libkg_gfx950.so"

KG_ARG_MEMORY = 1
KG_ARG_INT = 2
KG_ARG_FLOAT = 3

DTYPE_CODES = {
    "float32": 1,
    "float64": 2,
    "int32": 3,
    "int64": 4,
    "float16": 5,
    "bfloat16": 6,
}

ENTRY_POINTS = (
    "kg_gfx950_matmul_entry",
    "kg_gfx950_conv2d_entry",
    "kg_gfx950_flash_attention_entry",
)
CONTROL_SYMBOLS = (
    "kg_gfx950_set_launch_mode",
    "kg_gfx950_last_error",
    "kg_gfx950_abi_version",
    "kg_gfx950_cost",
    "kg_gfx950_fail",
    "kg_gfx950_check_memory_slot",
    "kg_gfx950_launch_stream",
    "kg_gfx950_launch_synchronous",
    "kg_gfx950_finish_launch",
)

# kg_gfx950_cost: op codes (KG_OP_*) and the order of its output array (KG_COST_*).
COST_OPS = {"matmul": 1, "conv2d": 2, "flash_attention": 3}
COST_KINDS = ("MAC", "MFMA", "HBM_READ", "HBM_WRITE", "MFMA_CYCLES")


class KgArgSlot(ctypes.Structure):
    """C slot, identical in layout to the reference's ``_CArgSlot``."""

    _fields_ = [
        ("kind", ctypes.c_int),
        ("data", ctypes.c_void_p),
        ("shape", ctypes.POINTER(ctypes.c_longlong)),
        ("stride", ctypes.POINTER(ctypes.c_longlong)),
        ("rank", ctypes.c_ulonglong),
        ("dtype_code", ctypes.c_int),
        ("int_value", ctypes.c_longlong),
        ("float_value", ctypes.c_double),
    ]


class NativeLibraryError(RuntimeError):
    """libkg_gfx950.so is missing or an entry point returned non-zero."""

    def __init__(self, message: str, status: int = 0) -> None:
        super().__init__(message)
        self.status = status


_LIBRARY: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("KG_GFX950_LIBRARY")
    return Path(override) if override else LIBRARY_PATH


def load_library() -> ctypes.CDLL:
    """Load (once) and return the gfx950 library; raise if it has not been built."""

    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    path = library_path()
    if not path.is_file():
        raise NativeLibraryError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    # torch ships its own libamdhip64.so.7. Loaded first, it serves this library too (same
    # soname); loaded after this library, it would be a second HIP runtime in the process,
    # and device memory or kernels of one are not valid in the other.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(path))
    for name in ENTRY_POINTS:
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.POINTER(KgArgSlot), ctypes.c_ulonglong]
        fn.restype = ctypes.c_int
    lib.kg_gfx950_set_launch_mode.argtypes = [ctypes.c_int, ctypes.c_void_p]
    lib.kg_gfx950_set_launch_mode.restype = ctypes.c_int
    lib.kg_gfx950_last_error.argtypes = []
    lib.kg_gfx950_last_error.restype = ctypes.c_char_p
    lib.kg_gfx950_abi_version.argtypes = []
    lib.kg_gfx950_abi_version.restype = ctypes.c_int
    lib.kg_gfx950_cost.argtypes = [ctypes.c_int, ctypes.POINTER(KgArgSlot), ctypes.c_ulonglong,
                                   ctypes.POINTER(ctypes.c_longlong)]
    lib.kg_gfx950_cost.restype = ctypes.c_int
    _LIBRARY = lib
    return lib


class TensorSpec:
    """Shape, element strides and dtype of an operand, for cost queries without memory.

    ``data_ptr()`` returns a non-zero placeholder: a present memory slot needs a non-NULL
    pointer, and kg_gfx950_cost never dereferences it.
    """

    def __init__(self, shape: Sequence[int], dtype: str, strides: Sequence[int] | None = None) -> None:
        self.shape = tuple(int(d) for d in shape)
        self.dtype = str(dtype).replace("torch.", "")
        if strides is None:
            strides, step = [], 1
            for d in reversed(self.shape):
                strides.insert(0, step)
                step *= max(d, 1)
        self._strides = tuple(int(s) for s in strides)

    @classmethod
    def of(cls, value: Any) -> "TensorSpec":
        """Spec of a torch tensor or numpy array (numpy byte strides become element strides)."""

        if hasattr(value, "stride") and callable(value.stride):
            return cls(value.shape, str(value.dtype), value.stride())
        itemsize = int(value.itemsize)
        return cls(value.shape, value.dtype.name, [s // itemsize for s in value.strides])

    def stride(self) -> tuple[int, ...]:
        return self._strides

    def data_ptr(self) -> int:
        return 256


def dtype_code_of(value: Any) -> int:
    name = str(getattr(value, "dtype", "")).replace("torch.", "")
    code = DTYPE_CODES.get(name)
    if code is None:
        raise NativeLibraryError(f"unsupported memory dtype {name!r}", -1)
    return code


def _is_memory(value: Any) -> bool:
    return hasattr(value, "data_ptr") and hasattr(value, "shape") and hasattr(value, "stride")


def marshal_slots(args: Sequence[Any]) -> tuple[ctypes.Array, list[Any]]:
    """Build the C slot array for ``args`` (tensors / None / int / float)."""

    slots: list[KgArgSlot] = []
    keepalive: list[Any] = []
    for position, arg in enumerate(args):
        if arg is None:
            shape = (ctypes.c_longlong * 1)(0)
            stride = (ctypes.c_longlong * 1)(1)
            keepalive.extend([shape, stride])
            slots.append(KgArgSlot(KG_ARG_MEMORY, None, shape, stride, 1, 0, 0, 0.0))
        elif isinstance(arg, bool):
            raise NativeLibraryError(f"bool runtime arg at position {position} is not supported", -1)
        elif isinstance(arg, Integral):
            slots.append(KgArgSlot(KG_ARG_INT, None, None, None, 0, 0, int(arg), 0.0))
        elif isinstance(arg, Real):
            slots.append(KgArgSlot(KG_ARG_FLOAT, None, None, None, 0, 0, 0, float(arg)))
        elif _is_memory(arg):
            dims = tuple(int(d) for d in arg.shape)
            strides = tuple(int(s) for s in arg.stride())
            shape = (ctypes.c_longlong * max(len(dims), 1))(*dims)
            stride = (ctypes.c_longlong * max(len(strides), 1))(*strides)
            keepalive.extend([shape, stride, arg])
            slots.append(
                KgArgSlot(KG_ARG_MEMORY, ctypes.c_void_p(int(arg.data_ptr())), shape, stride, len(dims), dtype_code_of(arg), 0, 0.0)
            )
        else:
            raise NativeLibraryError(f"unsupported runtime arg at position {position}: {type(arg).__name__}", -1)
    array = (KgArgSlot * max(len(slots), 1))(*slots)
    keepalive.append(array)
    return array, keepalive


def call_entry(entry_point: str, args: Sequence[Any], *, check: bool = True) -> int:
    """Invoke one gfx950 entry point with reference-ordered args; raise on non-zero if check."""

    lib = load_library()
    fn = getattr(lib, entry_point)
    array, keepalive = marshal_slots(args)
    status = int(fn(array, ctypes.c_ulonglong(len(args))))
    del keepalive
    if check and status != 0:
        detail = lib.kg_gfx950_last_error().decode("utf-8", "replace")
        raise NativeLibraryError(f"{entry_point} returned {status}: {detail}", status)
    return status


def cost(family: str, args: Sequence[Any]) -> dict[str, int]:
    """Per-call cost of ``family``'s entry on ``args`` (its full slot list; memory args may
    be TensorSpec), computed by kg_gfx950_cost without touching a GPU."""

    lib = load_library()
    op = COST_OPS.get(family)
    if op is None:
        raise NativeLibraryError(f"no cost model for {family!r}", -1)
    array, keepalive = marshal_slots(args)
    values = (ctypes.c_longlong * len(COST_KINDS))()
    status = int(lib.kg_gfx950_cost(op, array, ctypes.c_ulonglong(len(args)), values))
    del keepalive
    if status != 0:
        detail = lib.kg_gfx950_last_error().decode("utf-8", "replace")
        raise NativeLibraryError(f"kg_gfx950_cost({family}) returned {status}: {detail}", status)
    return {kind: int(values[i]) for i, kind in enumerate(COST_KINDS)}


def last_error() -> str:
    return load_library().kg_gfx950_last_error().decode("utf-8", "replace")


def set_launch_mode(synchronous: bool, stream: int | None = None) -> None:
    """synchronous=True: each entry waits for its kernel. False: enqueue on ``stream``."""

    load_library().kg_gfx950_set_launch_mode(1 if synchronous else 0, ctypes.c_void_p(stream or 0))


def matmul(out, lhs, rhs, bias=None, *tiles: int) -> None:
    call_entry("kg_gfx950_matmul_entry", (out, lhs, rhs, bias, *tiles))


def conv2d(out, x, weight, bias, stride=(1, 1), dilation=(1, 1), padding=(0, 0, 0, 0), tiles=(),
           memory_stage: int | None = None) -> None:
    """padding = (top, bottom, left, right); memory_stage: the LDS stage count (with 5 tiles)."""

    if memory_stage is not None and len(tiles) != 5:
        tiles = (1, 1, 1, 1, 1)
    stage = () if memory_stage is None else (int(memory_stage),)
    call_entry("kg_gfx950_conv2d_entry", (out, x, weight, bias, *stride, *dilation, *padding, *tiles, *stage))


def flash_attention(out, q, k, v, br: int = 64, bc: int = 64, scale: float = 1.0, causal: bool = False,
                    memory_stage: int | None = None) -> None:
    """memory_stage: the K/V ring depth of the MFMA kernel (2, 3 or 4)."""

    stage = () if memory_stage is None else (int(memory_stage),)
    call_entry("kg_gfx950_flash_attention_entry",
               (out, q, k, v, int(br), int(bc), float(scale), int(bool(causal)), *stage))
