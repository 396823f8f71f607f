"""``gfx950-lowering``: the pipeline registered next to the reference's
``npu-demo-lowering`` / ``cuda-sm89-lowering`` (kernel_gen/pipeline/cuda_sm89_lowering.py:
159-223, registry kernel_gen/passes/registry.py:343).

It runs on the kernel IR the front end builds (dsl.mlir_gen) and applies, in order:

  kernel-aggregate{matmul-acc=true}   fold K-loop matmul + add into accumulating matmuls
                                       (kernel_gen/passes/kernel/kernel_aggregate.py:292)
  kernel-pattern-fuse                  map a recognised loop nest onto a hand-written
                                       gfx950 kernel (passes/fuse.py)
  multi-buffer{memory-stage=N}         (option) the LDS ring depth of the fused kernel (the
                                       GEMMs' operand rings, attention's K/V rings, the
                                       conv kernels' stage count), the gfx950 reading of
                                       MultiBufferAnalysisPass's memory_stage
                                       (kernel_gen/passes/memory/multi_buffer.py); a kernel
                                       the call selects that cannot take it fails with an
                                       error naming it
  arch-parallelize{target=gfx950}      the per-operation path's grid: the leading
                                       perfectly nested loops (arch_parallelize.py:637-680)
  attach-arch-information{target=gfx950}  the target's hardware description

The memory-plan passes of the reference are not needed: a fused kernel manages LDS and
registers itself, and the per-operation path sizes its tiles' workspace in the entry.
LoopSoftPipelinePass's prologue / steady loop / epilogue is what every hand-written
kernel already does, so that pass has no knob here.

Options: ``target`` (gfx950), ``memory_stage`` (2, 3 or 4; fused kernels) and
``fuse`` (default true; false keeps every kernel on the per-operation path).
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Callable

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..gen_kernel.per_op import parallel_loops
from ..ir import Func
from ..passes import FusedCall, kernel_aggregate, pattern_fuse
from ..target import get_target_hardware

_PIPELINES: dict[str, Callable[..., "PassManager"]] = {}


def _error(message: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.PIPELINE, message)


def register_pipeline(name: str):
    def deco(fn):
        if name in _PIPELINES:
            raise _error(f"duplicate pipeline {name}")
        _PIPELINES[name] = fn
        return fn

    return deco


def get_pipeline(name: str, options: dict | None = None) -> "PassManager":
    builder = _PIPELINES.get(name)
    if builder is None:
        raise _error(f"unknown pipeline {name!r}")
    return builder(options)


@dataclass
class LoweredKernel:
    func: Func
    fused: FusedCall | None = None
    memory_stage: int | None = None
    parallel: tuple[str, ...] = ()
    hardware: dict[str, int] = field(default_factory=dict)
    applied: tuple[str, ...] = ()
    folds: int = 0


@dataclass
class PassManager:
    name: str
    passes: list[tuple[str, Callable[[LoweredKernel], LoweredKernel]]] = field(default_factory=list)

    def add_pass(self, name: str, fn: Callable[[LoweredKernel], LoweredKernel]) -> None:
        self.passes.append((name, fn))

    def run(self, func: Func) -> LoweredKernel:
        if not isinstance(func, Func):
            raise _error(f"{self.name} runs on kernel IR (dsl.mlir_gen)")
        state = LoweredKernel(func)
        for name, fn in self.passes:
            state = fn(state)
            state = replace(state, applied=state.applied + (name,))
        return state


def _kernel_aggregate(state: LoweredKernel) -> LoweredKernel:
    return replace(state, folds=state.folds + kernel_aggregate(state.func))


def _pattern_fuse(state: LoweredKernel) -> LoweredKernel:
    return replace(state, fused=pattern_fuse(state.func))


def _multi_buffer(stage: int) -> Callable[[LoweredKernel], LoweredKernel]:
    def run(state: LoweredKernel) -> LoweredKernel:
        if state.fused is None:
            # per-operation kernels stage nothing through LDS: like the reference pass on
            # IR it cannot ring, left alone
            return state
        return replace(state, memory_stage=stage)

    return run


def _arch_parallelize(state: LoweredKernel) -> LoweredKernel:
    if state.fused is not None:
        return state
    return replace(state, parallel=tuple(loop.attrs["iv"] for loop in parallel_loops(state.func)))


def _attach_arch_information(state: LoweredKernel) -> LoweredKernel:
    keys = ("block_num", "thread_num", "subthread_num", "sm_memory_size")
    return replace(state, hardware={k: get_target_hardware("gfx950", k) for k in keys})


def _flag(value, name: str) -> bool:
    text = str(value).strip().lower()
    if text in ("1", "true", "yes", "on"):
        return True
    if text in ("0", "false", "no", "off"):
        return False
    raise _error(f"gfx950-lowering {name} expects a bool, got {value!r}")


@register_pipeline("gfx950-lowering")
def build_gfx950_lowering_pipeline(options: dict | None = None) -> PassManager:
    opts = {} if options is None else dict(options)
    unknown = sorted(set(opts) - {"target", "memory_stage", "fuse"})
    if unknown:
        raise _error(f"gfx950-lowering accepts target, memory_stage and fuse options; got {', '.join(unknown)}")
    if opts.get("target", "gfx950") != "gfx950":
        raise _error("gfx950-lowering target must be gfx950")
    stage = None
    if "memory_stage" in opts:
        try:
            stage = int(opts["memory_stage"])
        except (TypeError, ValueError):
            stage = None
        if stage not in (2, 3, 4):
            raise _error(f"gfx950-lowering memory_stage must be 2, 3 or 4, got {opts['memory_stage']!r}")
    fuse = _flag(opts.get("fuse", True), "fuse")
    pm = PassManager(name="gfx950-lowering")
    pm.add_pass("kernel-aggregate{matmul-acc=true}", _kernel_aggregate)
    if fuse:
        pm.add_pass("kernel-pattern-fuse", _pattern_fuse)
    if stage is not None:
        pm.add_pass(f"multi-buffer{{memory-stage={stage}}}", _multi_buffer(stage))
    pm.add_pass("arch-parallelize{target=gfx950,parallel_level=block}", _arch_parallelize)
    pm.add_pass("attach-arch-information{target=gfx950}", _attach_arch_information)
    return pm
