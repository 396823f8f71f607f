"""Types the DSL kernels name (kernel_gen/symbol_variable of the reference): element types,
memory spaces, the SymbolDim annotation of INT parameters and the Memory annotation."""

from __future__ import annotations

from enum import Enum


class NumericType(Enum):
    Float32 = "f32"
    Float16 = "f16"
    BFloat16 = "bf16"


class MemorySpace(Enum):
    """On-chip spaces of the reference's npu_demo target (include/npu_demo/Arch.h:70-73);
    GM is global memory. gfx950 places every tile in per-workgroup global scratch."""

    GM = "GM"
    TSM = "TSM"
    TLM1 = "TLM1"
    TLM2 = "TLM2"


class SymbolDim:
    """Annotation of an INT kernel parameter (a runtime symbol, e.g. a tile size)."""


class Memory:
    """Annotation of a memory kernel parameter."""


__all__ = ["Memory", "MemorySpace", "NumericType", "SymbolDim"]
