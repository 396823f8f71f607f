"""Target registry in the reference's text format (kernel_gen/target/registry.py:41-51,
427-506, 671-702, 730, 862): ``name=``, ``arch.supported_ops=``, ``arch.unsupported_ops=``
and integer ``hw.<field>=`` lines; every ``targets/*.txt`` beside this file is loaded at
import. The reference's own target names are registered with their published specs so a
strategy can be looked up for any of them, and ``gfx950`` is added from targets/gfx950.txt."""

from __future__ import annotations

import re
from dataclasses import dataclass, field
from pathlib import Path

from ..core.error import ErrorKind, ErrorModule, KernelCodeError

ALLOWED_HARDWARE_FIELDS = frozenset(
    {
        "thread_num",
        "block_num",
        "subthread_num",
        "sm_memory_size",
        "lm_memory_size",
        "tsm_memory_size",
        "tlm1_memory_size",
        "tlm2_memory_size",
        "tlm3_memory_size",
    }
)
_NAME_RE = re.compile(r"^[a-z0-9_]+$")


@dataclass(frozen=True)
class TargetSpec:
    name: str
    supported_ops: frozenset[str] | None = None
    unsupported_ops: frozenset[str] = frozenset()
    hardware: dict[str, int] = field(default_factory=dict)


_TARGETS: dict[str, TargetSpec] = {}


def _error(message: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.TARGET, message)


def _ops(value: str) -> frozenset[str]:
    return frozenset(v.strip() for v in value.split(",") if v.strip())


def parse_target_txt(text: str, source: str = "<text>") -> TargetSpec:
    name = None
    supported: frozenset[str] | None = None
    unsupported: frozenset[str] = frozenset()
    hardware: dict[str, int] = {}
    for raw in text.splitlines():
        line = raw.strip()
        if not line or line.startswith("#"):
            continue
        if "=" not in line:
            raise _error(f"{source}: malformed line {raw!r}")
        key, value = (p.strip() for p in line.split("=", 1))
        if key == "name":
            name = value
        elif key == "arch.supported_ops":
            supported = _ops(value)
        elif key == "arch.unsupported_ops":
            unsupported = _ops(value)
        elif key.startswith("hw."):
            hw_key = key[3:]
            if hw_key not in ALLOWED_HARDWARE_FIELDS:
                raise _error(f"{source}: unknown hardware field {hw_key}")
            try:
                hardware[hw_key] = int(value)
            except ValueError as exc:
                raise _error(f"{source}: hw.{hw_key} must be an integer") from exc
        else:
            raise _error(f"{source}: unknown key {key}")
    if name is None or not _NAME_RE.match(name):
        raise _error(f"{source}: target name must match [a-z0-9_]+")
    if supported is not None and supported & unsupported:
        raise _error(f"{source}: ops both supported and unsupported")
    return TargetSpec(name, supported, unsupported, hardware)


def register_target(spec: TargetSpec) -> None:
    existing = _TARGETS.get(spec.name)
    if existing is not None and existing != spec:
        raise _error(f"target {spec.name} already registered with a different spec")
    _TARGETS[spec.name] = spec


def load_targets(directory: Path) -> dict[str, TargetSpec]:
    loaded = {}
    for path in sorted(Path(directory).glob("*.txt")):
        spec = parse_target_txt(path.read_text(), str(path))
        register_target(spec)
        loaded[spec.name] = spec
    return loaded


def get_target_spec(target: str) -> TargetSpec:
    spec = _TARGETS.get(target)
    if spec is None:
        raise _error(f"unknown target {target!r}")
    return spec


def is_registered(target: str) -> bool:
    return target in _TARGETS


def get_target_hardware(target: str, key: str) -> int | None:
    if key not in ALLOWED_HARDWARE_FIELDS:
        raise _error(f"unknown hardware field {key}")
    return get_target_spec(target).hardware.get(key)


def is_arch_op_supported(target: str, op_name: str) -> bool:
    spec = get_target_spec(target)
    if op_name in spec.unsupported_ops:
        return False
    return True if spec.supported_ops is None else op_name in spec.supported_ops


# The reference's built-in targets (kernel_gen/target/targets/{cpu,npu_demo,cuda_sm89}.txt).
register_target(TargetSpec("cpu", frozenset(), frozenset({"arch.get_thread_id"}), {"thread_num": 1, "block_num": 1, "subthread_num": 1}))
register_target(TargetSpec("npu_demo", None, frozenset({"arch.launch_kernel"}),
                           {"block_num": 2, "thread_num": 1, "subthread_num": 1, "tsm_memory_size": 2097152,
                            "tlm1_memory_size": 524288, "tlm2_memory_size": 1048576, "tlm3_memory_size": 1048576}))
register_target(TargetSpec("cuda_sm89", None, frozenset({"arch.launch_kernel"}),
                           {"block_num": 1, "thread_num": 256, "subthread_num": 32, "sm_memory_size": 49152,
                            "tsm_memory_size": 49152}))
load_targets(Path(__file__).resolve().parent / "targets")
