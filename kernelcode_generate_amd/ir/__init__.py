"""The gfx950 kernel IR: symbolic integers (sym), memory values and operations (core)."""

from .core import (DTYPES, ELEMENT_BYTES, TORCH_DTYPE_NAMES, Cmp, FVal, Func, Mem, Op, Param, Present, format_func,
                   format_op, parents_of, walk_block)
from .sym import Sym, as_sym, interval, smax, smin, sym_bin

__all__ = ["DTYPES", "ELEMENT_BYTES", "TORCH_DTYPE_NAMES", "Cmp", "FVal", "Func", "Mem", "Op", "Param", "Present",
           "Sym", "as_sym", "format_func", "format_op", "interval", "parents_of", "smax", "smin", "sym_bin",
           "walk_block"]
