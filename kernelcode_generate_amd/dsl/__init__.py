"""DSL front end of the gfx950 backend (the reference's kernel_gen/dsl/ast + mlir_gen)."""

from .mlir_gen import REFERENCE_MODULES, mlir_gen, mlir_gen_source, source_namespace

__all__ = ["REFERENCE_MODULES", "mlir_gen", "mlir_gen_source", "source_namespace"]
