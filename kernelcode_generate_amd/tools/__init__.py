"""Caller-side tools: dsl_run for the gfx950 target."""

from .dsl_run import DslRunResult, dsl_run

__all__ = ["DslRunResult", "dsl_run"]
