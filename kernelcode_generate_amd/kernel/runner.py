"""Demo runner for the gfx950 target, mirroring kernel/runner.py:201-278 of the reference:

- ``run_gfx950_demo(case_name, kernel_fn, real_args, output, expected, atol, rtol)`` is
  ``run_numpy_demo`` with target ``gfx950`` and pipeline ``gfx950-lowering``: set the
  target and dump dir, ``dsl_run``, write ``source.hip``, compare ``output`` with
  ``expected`` (np.allclose, default atol = rtol = 1e-4), restore the config;
- ``run_lowering_demo(case_name, kernel_fn, *compile_args)`` (:247-278) returns the lowered
  kernel and the generated source without executing; ``compile_args`` stand for the
  runtime arguments (arrays, tensors or native.TensorSpec for memory, ints, floats, None).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path
from typing import Any, Callable

import numpy as np

from ..core.config import restore_config, set_dump_dir, set_target, snapshot_config
from ..dsl import mlir_gen
from ..gen_kernel import gen_kernel
from ..pipeline import build_gfx950_lowering_pipeline
from ..tools.dsl_run import DslRunResult, dsl_run

KERNEL_DUMP_ROOT = Path("kernel_dump")


@dataclass(frozen=True)
class KernelDemoResult:
    case_name: str
    dsl_result: DslRunResult
    max_abs_diff: float
    atol: float
    rtol: float


def _to_numpy(value: Any) -> np.ndarray:
    if isinstance(value, np.ndarray):
        return value
    return value.detach().float().cpu().numpy()


def run_gfx950_demo(case_name: str, kernel_fn: Callable, real_args, output, expected, *, atol: float = 1e-4,
                    rtol: float = 1e-4, dump_root: Path | None = None) -> KernelDemoResult:
    snapshot = snapshot_config()
    try:
        set_target("gfx950")
        set_dump_dir((dump_root or KERNEL_DUMP_ROOT) / case_name.replace("/", "_")) if dump_root else set_dump_dir(None)
        result = dsl_run(kernel_fn, tuple(real_args), "gfx950-lowering")
        if not result.execute_result.ok:
            raise RuntimeError(f"{case_name}: dsl_run execute failed: {result.execute_result.failure_phrase}")
        got = _to_numpy(output).astype(np.float64)
        exp = _to_numpy(expected).astype(np.float64)
        max_abs_diff = float(np.max(np.abs(got - exp))) if got.size else 0.0
        if not np.allclose(got, exp, atol=atol, rtol=rtol):
            raise AssertionError(f"{case_name}: gfx950 output does not match reference "
                                 f"(max_abs_diff={max_abs_diff}, atol={atol}, rtol={rtol})")
        return KernelDemoResult(case_name, result, max_abs_diff, atol, rtol)
    finally:
        restore_config(snapshot)


def run_lowering_demo(case_name: str, kernel_fn: Callable, *compile_args):
    snapshot = snapshot_config()
    try:
        set_target("gfx950")
        lowered = build_gfx950_lowering_pipeline().run(mlir_gen(kernel_fn, compile_args))
        return lowered, gen_kernel(lowered)
    finally:
        restore_config(snapshot)
