"""Pipeline registry and the gfx950-lowering pipeline."""

from .gfx950_lowering import PassManager, build_gfx950_lowering_pipeline, get_pipeline, register_pipeline

__all__ = ["PassManager", "build_gfx950_lowering_pipeline", "get_pipeline", "register_pipeline"]
