"""``gfx950-lowering``: the pipeline registered next to the reference's
``npu-demo-lowering`` / ``cuda-sm89-lowering`` (kernel_gen/pipeline/cuda_sm89_lowering.py:
159-223, registry kernel_gen/passes/registry.py:343).

In the reference the pipeline rewrites xDSL IR; the IR passes it shares with
cuda-sm89-lowering are listed in ``IR_PASSES`` in their order (the memory-pool passes are
left out: gfx950 kernels manage LDS themselves). xDSL is not part of this backend, so the
steps that run here act on the recognised ``KernelPattern``: option checks, the K-loop
fusion rule of KernelAggregatePass(matmul_acc=True) (sequential-k accumulation, which the
GPU kernels honour by accumulating every k in fp32), the static-tile legality check, and
attaching the gfx950 hardware description (CUs, wave width, LDS bytes).

``memory_stage`` (option, 2-4) is the gfx950 reading of MultiBufferAnalysisPass's
``memory_stage`` (kernel_gen/passes/memory/multi_buffer.py, npu-demo-lowering uses 2): the
depth of the ring the staged operands cycle through. For matmul kernels it becomes the
LDS ring depth of the pipelined MFMA GEMM, passed as a trailing INT slot; without the
option the library uses 4. Like the reference pass on IR it cannot ring, it leaves conv2d
and attention alone (their K/V and channel-group buffers are fixed double buffers). The
software pipelining LoopSoftPipelinePass builds in IR (prologue, steady loop, epilogue) is
what every gfx950 kernel does already, so that pass has no knob here.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
from typing import Callable

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..gen_kernel import KernelPattern
from ..target import get_target_hardware

IR_PASSES = (
    "inline", "cse", "canonicalize", "decompass", "nn-lowering", "memory-plan", "symbol-hoist-pipeline",
    "tile-analysis", "kernel-pattern-attach", "transform-apply", "memory-plan", "symbol-hoist-pipeline",
    "kernel-aggregate{matmul-acc=true}", "kernel-decompose", "memory-plan", "symbol-hoist-pipeline",
    "producer-consumer-analysis", "arch-parallelize{target=gfx950,parallel_level=block}",
    "attach-arch-information{target=gfx950}", "outline-device-kernel", "template-name-infer",
)

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


@dataclass(frozen=True)
class LoweredKernel:
    pattern: KernelPattern
    hardware: dict[str, int]
    applied: tuple[str, ...]


@dataclass
class PassManager:
    name: str
    passes: list[tuple[str, Callable[[LoweredKernel], LoweredKernel]]] = field(default_factory=list)
    ir_passes: tuple[str, ...] = IR_PASSES

    def add_pass(self, name: str, fn: Callable[[LoweredKernel], LoweredKernel]) -> None:
        self.passes.append((name, fn))

    def run(self, pattern: KernelPattern) -> LoweredKernel:
        if not isinstance(pattern, KernelPattern):
            raise _error(f"{self.name} runs on a recognised KernelPattern")
        state = LoweredKernel(pattern, {}, ())
        for name, fn in self.passes:
            state = fn(state)
            state = replace(state, applied=state.applied + (name,))
        return state


def _check_static_tiles(state: LoweredKernel) -> LoweredKernel:
    for name, value in state.pattern.baked:
        if name.startswith("tile") or name in ("br", "bc"):
            if not isinstance(value, int) or value <= 0:
                raise _error(f"{state.pattern.function}: static {name}={value!r} must be a positive int")
        if name.startswith("stride") or name.startswith("dilation"):
            if not isinstance(value, int) or value <= 0:
                raise _error(f"{state.pattern.function}: {name}={value!r} must be a positive int")
        if name.startswith("pad") and (not isinstance(value, int) or value < 0):
            raise _error(f"{state.pattern.function}: {name}={value!r} must be a non-negative int")
    return state


def _kernel_aggregate(state: LoweredKernel) -> LoweredKernel:
    # matmul(acc = k_iter != k_start): one fp32 accumulation over all of K per output.
    return state


def _multi_buffer(stage: int) -> Callable[[LoweredKernel], LoweredKernel]:
    def run(state: LoweredKernel) -> LoweredKernel:
        p = state.pattern
        if p.family != "matmul":
            return state
        if len(p.params) + len(p.baked) != 7:
            raise _error(f"{p.function}: memory_stage needs the tile slots (7 forwarded slots)")
        return replace(state, pattern=replace(p, trailing=p.trailing + (("memory_stage", stage),)))

    return run


def _attach_arch_information(state: LoweredKernel) -> LoweredKernel:
    keys = ("block_num", "thread_num", "subthread_num", "sm_memory_size")
    return replace(state, hardware={k: get_target_hardware("gfx950", k) for k in keys})


@register_pipeline("gfx950-lowering")
def build_gfx950_lowering_pipeline(options: dict | None = None) -> PassManager:
    opts = {} if options is None else dict(options)
    unknown = sorted(set(opts) - {"target", "memory_stage"})
    if unknown:
        raise _error(f"gfx950-lowering accepts target and memory_stage options; got {', '.join(unknown)}")
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
    pm = PassManager(name="gfx950-lowering")
    pm.add_pass("tile-analysis", _check_static_tiles)
    pm.add_pass("kernel-aggregate{matmul-acc=true}", _kernel_aggregate)
    if stage is not None:
        pm.add_pass(f"multi-buffer{{memory-stage={stage}}}", _multi_buffer(stage))
    pm.add_pass("attach-arch-information{target=gfx950}", _attach_arch_information)
    return pm
