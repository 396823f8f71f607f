"""Target registry: text specs loaded from targets/*.txt (kernel_gen/target/registry.py)."""

from .registry import TargetSpec, get_target_hardware, get_target_spec, is_arch_op_supported, load_targets, register_target

__all__ = ["TargetSpec", "get_target_hardware", "get_target_spec", "is_arch_op_supported", "load_targets", "register_target"]
