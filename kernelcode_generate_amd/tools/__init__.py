"""Caller-side tools: dsl_run and dsl_cost_run for the gfx950 target."""

from .dsl_run import VALID_DSL_COST_KINDS, DslRunResult, dsl_cost_run, dsl_run, roofline_ns

__all__ = ["DslRunResult", "VALID_DSL_COST_KINDS", "dsl_cost_run", "dsl_run", "roofline_ns"]
