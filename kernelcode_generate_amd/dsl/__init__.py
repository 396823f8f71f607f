"""DSL front end of the gfx950 backend (the reference's kernel_gen/dsl/ast + mlir_gen)."""

from .mlir_gen import mlir_gen

__all__ = ["mlir_gen"]
