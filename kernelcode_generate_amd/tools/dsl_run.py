"""``dsl_run(func_obj, real_args, pipeline)`` for the gfx950 target
(kernel_gen/tools/dsl_run.py:578-653): check the configured target and the arity against
the kernel's signature, build the kernel's IR from its Python source (dsl.mlir_gen, the
reference's mlir_gen), run the pipeline (gfx950-lowering), generate the SourceBundle,
compile it through ``ExecutionEngine("gfx950")`` and execute it with the real arguments.

Memory arguments may be ROCm torch tensors (used in place) or host numpy arrays /
CPU tensors, which are staged to the device and copied back after the call -- what the
reference's cuda_sm89 entry does per call (source_bundle.py:647-707). ``None`` is
allowed for memory parameters the kernel tests with `is None` / `is not None`; ints and
floats are passed as INT / FLOAT slots.

``dsl_cost_run(func_obj, real_args, pipeline, cost_kind)`` (kernel_gen/tools/dsl_run.py:
656-730) returns one integer cost of the same call without running it: the reference
lowers to an npu_demo cost function whose kinds are DMA1..DMA4, MAC, VECTOR1, VECTOR2;
here the library's kg_gfx950_cost runs the fused kernel's validation and kernel choice and
reports MAC, MFMA (wave-level matrix instructions of the chosen kernel), HBM_READ and
HBM_WRITE (compulsory bytes), and ROOFLINE_NS is the time those imply at MI355X's peaks
(the lower bound any run of the call meets). Kernels on the per-operation path have no
cost model.
"""

from __future__ import annotations

import atexit
import inspect
from dataclasses import dataclass
from numbers import Integral, Real
from pathlib import Path
from typing import Any, Callable

from ..core.config import get_dump_dir, get_target
from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..dsl import mlir_gen
from ..execute_engine import CompiledKernel, ExecuteResult, ExecutionEngine
from ..gen_kernel import gen_kernel, library_slots
from ..ir import Sym
from ..passes import FusedCall
from ..pipeline import PassManager, get_pipeline
from ..pipeline.gfx950_lowering import LoweredKernel

ARITY_ERROR = "DslRunArityMismatch: real_args count must match the kernel's positional parameters"
VALID_DSL_COST_KINDS = ("MAC", "MFMA", "HBM_READ", "HBM_WRITE", "MFMA_CYCLES", "ROOFLINE_NS")
DSL_COST_KIND_ERROR = ("DslCostRunInvalidCostKind: cost_kind must be one of [MAC, MFMA, HBM_READ, HBM_WRITE, "
                       "MFMA_CYCLES, ROOFLINE_NS]")
# MI355X: 256 CUs x 4 SIMDs at 2.4 GHz (the library reports the SIMD cycles its MFMAs occupy:
# 16 per 16x16x32 and 32 per 32x32x16 bf16/f16 MFMA, 64 per 32x32x2 fp32 MFMA); HBM3E moves
# 8 TB/s (8000 bytes per ns).
SIMDS, CLOCK_GHZ, HBM_BYTES_PER_NS = 1024, 2.4, 8000.0


def roofline_ns(costs: dict) -> int:
    """The time below which no kernel can finish the call: the larger of its matrix-core
    time (the chosen kernel's MFMA instructions x the cycles each occupies, spread over every
    SIMD at the peak clock) and its compulsory HBM traffic at peak bandwidth, in ns (rounded
    up)."""

    mfma_ns = costs["MFMA_CYCLES"] / SIMDS / CLOCK_GHZ
    hbm_ns = (costs["HBM_READ"] + costs["HBM_WRITE"]) / HBM_BYTES_PER_NS
    return int(-(-max(mfma_ns, hbm_ns) // 1))
DSL_COST_TARGET_ERROR = "DslCostRunInvalidTarget: dsl_cost_run only supports target 'gfx950'"
DSL_COST_OUTPUT_ERROR = "DslCostRunInvalidOutput: cost query was rejected by the gfx950 library"
_COMPILED: dict[str, CompiledKernel] = {}


@atexit.register
def _close_cached() -> None:
    for kernel in _COMPILED.values():
        try:
            kernel.close()
        except Exception:
            pass
    _COMPILED.clear()


@dataclass(frozen=True)
class DslRunResult:
    fused: FusedCall | None
    module: LoweredKernel
    source: str
    compiled_kernel: CompiledKernel
    execute_result: ExecuteResult
    runtime_args: tuple


def _error(message: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.TOOLS, message)


def _dtype_name(value: Any) -> str:
    return str(getattr(value, "dtype", "")).replace("torch.", "")


def _stage(arg: Any):
    """Return (device tensor, writeback callable or None) for one memory argument."""

    import numpy as np
    import torch

    if isinstance(arg, np.ndarray):
        if arg.dtype.name not in ("float32", "float16"):
            raise _error(f"unsupported numpy dtype {arg.dtype}")
        dev = torch.from_numpy(np.ascontiguousarray(arg)).to("cuda")

        def back(host=arg, d=dev):
            host[...] = d.cpu().numpy()

        return dev, back
    if isinstance(arg, torch.Tensor) and arg.device.type != "cuda":
        dev = arg.contiguous().to("cuda")

        def back(host=arg, d=dev):
            host.copy_(d.cpu())

        return dev, back
    return arg, None


def _resolve_pipeline(pipeline: str | PassManager) -> PassManager:
    if isinstance(pipeline, PassManager):
        return pipeline
    if isinstance(pipeline, str):
        return get_pipeline(pipeline)
    raise _error("pipeline must be a registered name or a PassManager")


def _check_arity(func_obj: Callable, real_args: tuple | list) -> tuple:
    if not isinstance(real_args, (tuple, list)):
        raise _error("real_args must be a tuple or list")
    args = tuple(real_args)
    params = [p for p in inspect.signature(func_obj).parameters.values()
              if p.kind in (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)]
    if len(args) != len(params):
        raise _error(ARITY_ERROR)
    return args


def _is_scalar(arg: Any) -> bool:
    return arg is None or isinstance(arg, (Integral, Real))


def lower(func_obj: Callable, args: tuple, pipeline: str | PassManager) -> LoweredKernel:
    """Front end + pipeline: the lowered kernel for these runtime argument kinds."""

    return _resolve_pipeline(pipeline).run(mlir_gen(func_obj, args))


def dsl_run(func_obj: Callable, real_args: tuple | list, pipeline: str | PassManager) -> DslRunResult:
    target = get_target()
    if target != "gfx950":
        raise _error(f"DslRunInvalidTarget: core config target must be 'gfx950' for this backend, got {target!r}")
    args = _check_arity(func_obj, real_args)
    lowered = lower(func_obj, args, pipeline)
    source = gen_kernel(lowered)
    dump = get_dump_dir()
    if dump is not None:
        out_dir = Path(dump) / lowered.func.name
        out_dir.mkdir(parents=True, exist_ok=True)
        (out_dir / "source.hip").write_text(source)
    compiled = _COMPILED.get(source)
    if compiled is None:
        compiled = ExecutionEngine(target="gfx950").compile(source=source, function=lowered.func.name)
        _COMPILED[source] = compiled
    staged = []
    writebacks = []
    for a in args:
        if _is_scalar(a):
            staged.append(a)
            continue
        dev, back = _stage(a)
        staged.append(dev)
        if back is not None:
            writebacks.append(back)
    result = compiled.execute(args=tuple(staged))
    for back in writebacks:
        back()
    return DslRunResult(fused=lowered.fused, module=lowered, source=source, compiled_kernel=compiled,
                        execute_result=result, runtime_args=tuple(staged))


def _evaluate(expr: Sym, func, args: tuple) -> int:
    index = {p.name: i for i, p in enumerate(func.params)}

    def leaf(s: Sym) -> int:
        value = args[index[s.args[0]]]
        if s.op == "arg":
            return int(value)
        if s.op == "dim":
            return int(tuple(value.shape)[s.args[1]])
        raise _error("fused operands cannot use loop indices")

    return expr.evaluate(leaf)


def dsl_cost_run(func_obj: Callable, real_args: tuple | list, pipeline: str | PassManager, cost_kind: str) -> int:
    """One integer cost of ``func_obj(*real_args)`` on gfx950, computed without a GPU.

    Contract of kernel_gen/tools/dsl_run.py:656-730: ``cost_kind`` is required and checked
    first, then the target, the pipeline and the arity; the result is an int. Memory
    arguments contribute only shape, strides and dtype (torch tensors on any device, numpy
    arrays or native.TensorSpec), so full-size shapes cost nothing to query.
    """

    from .. import native

    if cost_kind not in VALID_DSL_COST_KINDS:
        raise _error(DSL_COST_KIND_ERROR)
    if get_target() != "gfx950":
        raise _error(DSL_COST_TARGET_ERROR)
    pm = _resolve_pipeline(pipeline)
    args = _check_arity(func_obj, real_args)
    lowered = pm.run(mlir_gen(func_obj, args))
    if lowered.fused is None:
        raise _error(f"{DSL_COST_OUTPUT_ERROR}: {lowered.func.name} runs on the per-operation path, which has no "
                     "cost model")
    index = {p.name: i for i, p in enumerate(lowered.func.params)}
    slots = []
    for kind, value in library_slots(lowered.fused, lowered.memory_stage):
        if kind == "mem":
            arg = None if value is None else args[index[value]]
            slots.append(None if arg is None else native.TensorSpec.of(arg))
        elif kind == "int":
            slots.append(_evaluate(value, lowered.func, args))
        else:
            slots.append(float(args[index[value.arg]]) if value.arg is not None else float(value.value))
    try:
        costs = native.cost(lowered.fused.family, slots)
    except native.NativeLibraryError as exc:
        raise _error(f"{DSL_COST_OUTPUT_ERROR}: {exc}") from exc
    if cost_kind == "ROOFLINE_NS":
        return roofline_ns(costs)
    return costs[cost_kind]
