"""gfx950 source generation: lowered kernel IR -> SourceBundle.

The reference's emitter walks a lowered module and writes target source
(kernel_gen/dsl/gen_kernel/gen_kernel.py:150-180; per-target packages registered through
``@emit_c_impl(ModuleOp, target=...)``, emit/register.py:187-215, 356) and, for its GPU
target, a SourceBundle of files introduced by ``// __KG_BUNDLE_FILE__:<path>`` lines
(emit/register.py:69). The gfx950 emitter writes a bundle whose ``kernel.hip`` defines the
reference's entry ``extern "C" int kg_execute_entry(const _ArgSlot*, u64)`` in one of two
forms:

  - fused: kernel-pattern-fuse recognised the loop nest, and the entry forwards the
    kernel's own slots to the hand-written CDNA4 kernel's entry of libkg_gfx950.so, with
    the integer and float operands the nest implies (strides, pads, tiles, scale, causal)
    computed from the slots at run time;
  - per-operation: every other kernel, emitted by gen_kernel.per_op as one HIP kernel
    that executes the IR operation by operation on the workgroups of the GPU.

Both carry the reference's ``// kg.allow_absent_memory_args:`` metadata for memory
parameters that may be absent (runtime_args.py:497-516).
"""

from __future__ import annotations

import hashlib
import math

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..ir import FVal, Func, Sym, format_func
from ..passes import FusedCall
from .per_op import emit_per_op

BUNDLE_MARKER_PREFIX = "// __KG_BUNDLE_FILE__:"
ENTRY_POINT = "kg_execute_entry"
LIBRARY_ENTRY = {
    "matmul": "kg_gfx950_matmul_entry",
    "conv2d": "kg_gfx950_conv2d_entry",
    "flash_attention": "kg_gfx950_flash_attention_entry",
}
_DTYPE_NAMES = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def _error(message: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.GEN_KERNEL, message)


def library_slots(call: FusedCall, memory_stage: int | None = None) -> list:
    """The library entry's slot list as (kind, value): ("mem", param | None), ("int", Sym),
    ("float", FVal). A memory_stage becomes the entry's trailing ring-depth slot: matmul
    (out, lhs, rhs, bias, 3 tiles, stage), conv2d (out, x, w, bias, 8 geometry ints,
    5 tiles, stage), flash attention (out, q, k, v, br, bc, scale, causal, stage); without
    it matmul takes the 4-slot form and conv2d the 12-slot one."""

    slots: list = [("mem", name) for name in call.memory]
    if call.family == "matmul":
        if memory_stage is not None:
            tiles = call.tiles or (Sym.const(1),) * 3
            slots += [("int", t) for t in tiles] + [("int", Sym.const(memory_stage))]
        return slots
    slots += [("int", e) for e in call.ints]
    if call.family == "conv2d" and memory_stage is not None:
        slots += [("int", t) for t in (call.tiles or (Sym.const(1),) * 5)]
    slots += [("float", v) for v in call.floats]
    slots += [("int", e) for e in call.trailing_ints]
    if memory_stage is not None:
        slots.append(("int", Sym.const(memory_stage)))
    return slots


def _header(func: Func, kind: str, notes: list[str]) -> list[str]:
    digest = hashlib.sha256(format_func(func).encode()).hexdigest()[:16]
    lines = [f"{BUNDLE_MARKER_PREFIX}kernel.hip", f"// kg.gfx950.kernel: {func.name}", f"// kg.gfx950.path: {kind}",
             f"// kg.gfx950.ir_hash: {digest}"]
    lines += [f"// kg.gfx950.note: {n}" for n in notes]
    absent = [f"{i}:{_DTYPE_NAMES[p.dtype]}:{p.rank}" for i, p in enumerate(func.params) if p.kind == "memory" and p.optional]
    if absent:
        lines.append(f"// kg.allow_absent_memory_args: {';'.join(absent)}")
    return lines


def emit_fused(func: Func, call: FusedCall, memory_stage: int | None = None) -> str:
    index = {p.name: i for i, p in enumerate(func.params)}
    entry = LIBRARY_ENTRY[call.family]
    slots = library_slots(call, memory_stage)
    checks: list[str] = []

    def leaf(s: Sym) -> str:
        if s.op == "arg":
            i = index[s.args[0]]
            checks.append(f'  if (s[{i}].kind != KG_ARG_INT) return kg_gfx950_fail(-1, "slot {i} ({s.args[0]}): '
                          f'expected int slot");')
            return f"s[{i}].int_value"
        if s.op == "dim":
            i = index[s.args[0]]
            checks.append(f'  if (s[{i}].kind != KG_ARG_MEMORY || s[{i}].shape == nullptr || s[{i}].rank <= {s.args[1]}ULL) '
                          f'return kg_gfx950_fail(-1, "slot {i} ({s.args[0]}): expected a memory slot of rank > {s.args[1]}");')
            return f"s[{i}].shape[{s.args[1]}]"
        raise _error("fused operands cannot use loop indices")

    body: list[str] = []
    for k, (kind, value) in enumerate(slots):
        if kind == "mem":
            if value is None:
                body.append(f"  slots[{k}] = KgArgSlot{{}};  // absent")
                body.append(f"  slots[{k}].kind = KG_ARG_MEMORY; slots[{k}].shape = kZero; slots[{k}].stride = kOne; "
                            f"slots[{k}].rank = 1;")
            else:
                body.append(f"  slots[{k}] = s[{index[value]}];  // {value}")
        elif kind == "int":
            body.append(f"  slots[{k}] = KgArgSlot{{}};")
            body.append(f"  slots[{k}].kind = KG_ARG_INT; slots[{k}].int_value = {value.to_c(leaf)};")
        else:
            v: FVal = value
            body.append(f"  slots[{k}] = KgArgSlot{{}};")
            if v.arg is not None:
                i = index[v.arg]
                checks.append(f'  if (s[{i}].kind != KG_ARG_FLOAT && s[{i}].kind != KG_ARG_INT) return kg_gfx950_fail(-1, '
                              f'"slot {i} ({v.arg}): expected float slot");')
                body.append(f"  slots[{k}].kind = KG_ARG_FLOAT; slots[{k}].float_value = s[{i}].kind == KG_ARG_FLOAT ? "
                            f"s[{i}].float_value : (double)s[{i}].int_value;")
            else:
                lit = "HUGE_VAL" if math.isinf(v.value) and v.value > 0 else "-HUGE_VAL" if math.isinf(v.value) else repr(v.value)
                body.append(f"  slots[{k}].kind = KG_ARG_FLOAT; slots[{k}].float_value = {lit};")
    # memory parameters the call does not read must still be valid arguments
    for i, p in enumerate(func.params):
        if p.kind == "memory" and p.name not in call.memory:
            checks.append(f'  if (kg_gfx950_check_memory_slot(s, {i}, {p.rank}, {1 if p.optional else 0}, 0, "{p.name}") '
                          f'!= 0) return -1;')
    seen = set()
    uniq_checks = [c for c in checks if not (c in seen or seen.add(c))]
    notes = [f"fused: {entry}"] + list(call.notes)
    lines = _header(func, "fused", notes) + [
        "#include <cmath>",
        '#include "kg_gfx950.h"',
        '#include "gfx950/kg_tile.h"',
        "",
        "using kg_tile::kg_floordiv; using kg_tile::kg_max; using kg_tile::kg_min; using kg_tile::kg_mod;",
        "",
        f"// {func.name} as {ENTRY_POINT}: the {call.family} nest of this kernel runs as {entry}",
        f'extern "C" int {ENTRY_POINT}(const KgArgSlot* s, unsigned long long n) {{',
        "  static const long long kZero[1] = {0};",
        "  static const long long kOne[1] = {1};",
        "  (void)kZero; (void)kOne;",
        '  if (s == nullptr) return kg_gfx950_fail(-1, "ordered_args is null");',
        f'  if (n != {len(func.params)}ULL) return kg_gfx950_fail(-1, "{func.name} expects {len(func.params)} slots");',
        *uniq_checks,
        f"  KgArgSlot slots[{len(slots)}];",
        *body,
        f"  return {entry}(slots, {len(slots)}ULL);",
        "}",
        "",
    ]
    return "\n".join(lines)


def gen_kernel(lowered) -> str:
    """SourceBundle text of a lowered kernel (pipeline.LoweredKernel)."""

    func = lowered.func
    if lowered.fused is not None:
        return emit_fused(func, lowered.fused, lowered.memory_stage)
    return "\n".join(_header(func, "per-op", ["every operation on the workgroups (gfx950/kg_tile.h)"])) + "\n" + \
        emit_per_op(func, func.name)


__all__ = ["BUNDLE_MARKER_PREFIX", "ENTRY_POINT", "LIBRARY_ENTRY", "emit_fused", "emit_per_op", "gen_kernel",
           "library_slots"]
