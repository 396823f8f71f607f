"""gfx950 source generation for the three hot-path patterns.

The reference's emitter walks the lowered IR of a DSL kernel and writes target source
(kernel_gen/dsl/gen_kernel/gen_kernel.py:150-180; per-target packages registered through
``@emit_c_impl(ModuleOp, target=...)``, emit/register.py:187-215, 356). The gfx950 backend
recognises the three loop nests the demos lower to -- the K-loop ``kernel.matmul`` with
optional rank-1 bias, the ``img2col2d -> matmul -> transpose -> add`` conv nest, and the
online-softmax flash-attention nest -- and emits a SourceBundle whose ``kernel.hip``
defines the reference's entry ``extern "C" int kg_execute_entry(const _ArgSlot*, u64)``
as a call into the hand-written CDNA4 kernels of libkg_gfx950.so, appending the constants
the static demos bake into their bodies (tiles, strides, pads).

A ``KernelPattern`` is the recognised form of one DSL kernel: its family, parameter
order, the constants baked into it and which argument may be absent. Patterns are
registered per DSL function name (the nine demos of kernel/{matmul,conv2d,flash_attention}
plus the scaled / causal flash-attention variants the BASELINE configs need).
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Callable, Sequence

from ..core.error import ErrorKind, ErrorModule, KernelCodeError

BUNDLE_MARKER_PREFIX = "// __KG_BUNDLE_FILE__:"
ENTRY_POINT = "kg_execute_entry"
LIBRARY_ENTRY = {
    "matmul": ("kg_gfx950_matmul_entry", (4, 7, 8)),
    "conv2d": ("kg_gfx950_conv2d_entry", (12, 17)),
    "flash_attention": ("kg_gfx950_flash_attention_entry", (4, 6, 8)),
}


@dataclass(frozen=True)
class KernelPattern:
    family: str                                  # matmul | conv2d | flash_attention
    function: str                                # DSL function name
    params: tuple[str, ...]                      # DSL parameter order = slot order
    baked: tuple[tuple[str, int | float], ...]   # constants inserted after slot `insert_at`
    insert_at: int                               # index where baked constants go
    trailing: tuple[tuple[str, int | float], ...] = ()  # constants appended at the end
    absent_index: int | None = None              # optional memory arg (bias)
    absent_rank: int = 1
    dtype: str = "float32"
    notes: tuple[str, ...] = field(default_factory=tuple)

    @property
    def library_entry(self) -> str:
        return LIBRARY_ENTRY[self.family][0]

    @property
    def forwarded_count(self) -> int:
        return len(self.params) + len(self.baked) + len(self.trailing)


def _error(message: str) -> KernelCodeError:
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.GEN_KERNEL, message)


def _c_literal(value: int | float) -> tuple[str, str]:
    if isinstance(value, bool) or isinstance(value, int):
        return "KG_ARG_INT", f"{int(value)}LL"
    return "KG_ARG_FLOAT", repr(float(value))


def gen_kernel(pattern: KernelPattern) -> str:
    """SourceBundle text for one recognised kernel pattern."""

    entry, counts = LIBRARY_ENTRY[pattern.family]
    total = pattern.forwarded_count
    if total not in counts:
        raise _error(f"{pattern.function}: {total} forwarded slots do not match {entry} ({counts})")
    n_in = len(pattern.params)
    digest = hashlib.sha256(repr(pattern).encode()).hexdigest()[:16]
    lines = [
        f"{BUNDLE_MARKER_PREFIX}kernel.hip",
        f"// kg.gfx950.kernel: {pattern.function}",
        f"// kg.gfx950.pattern: {pattern.family}",
        f"// kg.gfx950.pattern_hash: {digest}",
        f"// kg.gfx950.library_entry: {entry}",
    ]
    lines += [f"// kg.gfx950.note: {note}" for note in pattern.notes]
    if pattern.absent_index is not None:
        lines.append(f"// kg.allow_absent_memory_args: {pattern.absent_index}:{pattern.dtype}:{pattern.absent_rank}")
    lines += [
        '#include "kg_gfx950.h"',
        "",
        f"// runtime entry for {pattern.function} as {ENTRY_POINT}",
        f'extern "C" int {ENTRY_POINT}(const KgArgSlot* ordered_args, unsigned long long arg_count) {{',
        "  if (ordered_args == nullptr) return -1;",
        f"  if (arg_count != {n_in}ULL) return -1;",
    ]
    if not pattern.baked and not pattern.trailing:
        lines.append(f"  return {entry}(ordered_args, arg_count);")
    else:
        lines.append(f"  KgArgSlot slots[{total}];")
        out = 0

        def const_slot(name: str, value: int | float) -> None:
            nonlocal out
            kind, lit = _c_literal(value)
            field_name = "int_value" if kind == "KG_ARG_INT" else "float_value"
            lines.append(f"  slots[{out}] = KgArgSlot{{}};  // {name}")
            lines.append(f"  slots[{out}].kind = {kind};")
            lines.append(f"  slots[{out}].{field_name} = {lit};")
            out += 1

        for i in range(pattern.insert_at):
            lines.append(f"  slots[{out}] = ordered_args[{i}];  // {pattern.params[i]}")
            out += 1
        for name, value in pattern.baked:
            const_slot(name, value)
        for i in range(pattern.insert_at, n_in):
            lines.append(f"  slots[{out}] = ordered_args[{i}];  // {pattern.params[i]}")
            out += 1
        for name, value in pattern.trailing:
            const_slot(name, value)
        lines.append(f"  return {entry}(slots, {total}ULL);")
    lines += ["}", ""]
    return "\n".join(lines)


def forward_args(pattern: KernelPattern, args: Sequence) -> tuple:
    """The slot list the generated entry forwards to the library entry for ``args``: the
    runtime args with the baked constants inserted at ``insert_at`` and the trailing
    constants appended (the same order gen_kernel writes into kernel.hip)."""

    args = tuple(args)
    if len(args) != len(pattern.params):
        raise _error(f"{pattern.function}: expected {len(pattern.params)} args, got {len(args)}")
    baked = tuple(value for _, value in pattern.baked)
    trailing = tuple(value for _, value in pattern.trailing)
    return args[: pattern.insert_at] + baked + args[pattern.insert_at:] + trailing


# ------------------------------------------------------------------------------------
# pattern registry (recognition by DSL function name)
# ------------------------------------------------------------------------------------

PatternBuilder = Callable[[dict, str], KernelPattern]
_PATTERNS: dict[str, PatternBuilder] = {}


def register_pattern(function_name: str, builder: PatternBuilder) -> None:
    _PATTERNS[function_name] = builder


def recognise(func_obj: Callable, dtype: str = "float32") -> KernelPattern:
    """Map a DSL kernel to its gfx950 pattern; module globals supply baked constants."""

    name = getattr(func_obj, "__name__", "")
    builder = _PATTERNS.get(name)
    if builder is None:
        raise _error(f"gfx950 has no pattern for DSL function {name!r}")
    return builder(getattr(func_obj, "__globals__", {}), dtype)


def known_patterns() -> tuple[str, ...]:
    return tuple(sorted(_PATTERNS))


def _g(globs: dict, key: str, default):
    value = globs.get(key, default)
    return value


_MATMUL_PARAMS = ("out", "lhs", "rhs", "bias")
_MATMUL_TILES = ("tile_h", "tile_w", "tile_k")
_CONV_PARAMS = ("out", "input_tensor", "weight", "bias")
_CONV_GEOM = ("stride_h", "stride_w", "dilation_h", "dilation_w", "pad_top", "pad_bottom", "pad_left", "pad_right")
_CONV_TILES = ("tile_f", "tile_c", "tile_n", "tile_ho", "tile_wo")
_FA_PARAMS = ("out", "q", "k", "v")


def _matmul_static_static(globs: dict, dtype: str) -> KernelPattern:
    # kernel/matmul/inputs_static_tile_static.py:56-110: tiles are module constants
    tiles = (_g(globs, "_TILE_M", 48), _g(globs, "_TILE_N", 80), _g(globs, "_TILE_K", 56))
    return KernelPattern("matmul", "matmul_inputs_static_tile_static_kernel", _MATMUL_PARAMS,
                         tuple(zip(("tile_m", "tile_n", "tile_k"), tiles)), 4, absent_index=3, dtype=dtype)


def _matmul_tile_dynamic(name: str) -> PatternBuilder:
    def build(globs: dict, dtype: str) -> KernelPattern:
        return KernelPattern("matmul", name, _MATMUL_PARAMS + _MATMUL_TILES, (), 7, absent_index=3, dtype=dtype)

    return build


def _conv_geometry(globs: dict) -> tuple[tuple[str, int], ...]:
    # the static conv demos hard-code stride 8 and take dilation/pads from module constants
    values = (8, 8, _g(globs, "_STATIC_DILATION_H", 1), _g(globs, "_STATIC_DILATION_W", 1),
              _g(globs, "_STATIC_PAD_TOP", 0), _g(globs, "_STATIC_PAD_BOTTOM", 0),
              _g(globs, "_STATIC_PAD_LEFT", 0), _g(globs, "_STATIC_PAD_RIGHT", 0))
    return tuple(zip(_CONV_GEOM, values))


def _conv_static_static(globs: dict, dtype: str) -> KernelPattern:
    tiles = (_g(globs, "_STATIC_TILE_F", 8), _g(globs, "_STATIC_TILE_C", 16), _g(globs, "_STATIC_TILE_N", 4),
             _g(globs, "_STATIC_TILE_HO", 8), _g(globs, "_STATIC_TILE_WO", 9))
    return KernelPattern("conv2d", "conv2d_inputs_static_tile_static_kernel", _CONV_PARAMS,
                         _conv_geometry(globs) + tuple(zip(_CONV_TILES, tiles)), 4, absent_index=3, dtype=dtype)


def _conv_static_dynamic(globs: dict, dtype: str) -> KernelPattern:
    return KernelPattern("conv2d", "conv2d_inputs_static_tile_dynamic_kernel", _CONV_PARAMS + _CONV_TILES,
                         _conv_geometry(globs), 4, absent_index=3, dtype=dtype)


def _conv_dynamic_dynamic(globs: dict, dtype: str) -> KernelPattern:
    return KernelPattern("conv2d", "conv2d_inputs_dynamic_tile_dynamic_kernel", _CONV_PARAMS + _CONV_GEOM + _CONV_TILES,
                         (), 17, absent_index=3, dtype=dtype)


def _fa_static_static(globs: dict, dtype: str) -> KernelPattern:
    tiles = (_g(globs, "_STATIC_BR", 64), _g(globs, "_STATIC_BC", 80))
    return KernelPattern("flash_attention", "flash_attention_inputs_static_tile_static_kernel", _FA_PARAMS,
                         tuple(zip(("br", "bc"), tiles)), 4, dtype=dtype)


def _fa_tile_dynamic(name: str) -> PatternBuilder:
    def build(globs: dict, dtype: str) -> KernelPattern:
        return KernelPattern("flash_attention", name, _FA_PARAMS + ("br", "bc"), (), 6, dtype=dtype)

    return build


def _fa_scaled(name: str, causal: bool) -> PatternBuilder:
    # scale = 1/sqrt(D) as a `kernel.mul` by a filled tile and, for causal, the
    # `min(seq, m0 + br)` key bound plus the 0/-inf diagonal mask: the BASELINE variants
    def build(globs: dict, dtype: str) -> KernelPattern:
        scale = float(_g(globs, "_SOFTMAX_SCALE", 0.0))
        return KernelPattern("flash_attention", name, _FA_PARAMS + ("br", "bc", "scale"), (), 7,
                             trailing=(("causal", 1 if causal else 0),), dtype=dtype,
                             notes=("scale = runtime FLOAT slot", "causal lower-triangular mask" if causal else "no mask"))

    return build


register_pattern("matmul_inputs_static_tile_static_kernel", _matmul_static_static)
register_pattern("matmul_inputs_static_tile_dynamic_kernel", _matmul_tile_dynamic("matmul_inputs_static_tile_dynamic_kernel"))
register_pattern("matmul_inputs_dynamic_tile_dynamic_kernel", _matmul_tile_dynamic("matmul_inputs_dynamic_tile_dynamic_kernel"))
register_pattern("conv2d_inputs_static_tile_static_kernel", _conv_static_static)
register_pattern("conv2d_inputs_static_tile_dynamic_kernel", _conv_static_dynamic)
register_pattern("conv2d_inputs_dynamic_tile_dynamic_kernel", _conv_dynamic_dynamic)
register_pattern("flash_attention_inputs_static_tile_static_kernel", _fa_static_static)
register_pattern("flash_attention_inputs_static_tile_dynamic_kernel",
                 _fa_tile_dynamic("flash_attention_inputs_static_tile_dynamic_kernel"))
register_pattern("flash_attention_inputs_dynamic_tile_dynamic_kernel",
                 _fa_tile_dynamic("flash_attention_inputs_dynamic_tile_dynamic_kernel"))
register_pattern("flash_attention_scaled_kernel", _fa_scaled("flash_attention_scaled_kernel", False))
register_pattern("flash_attention_scaled_causal_kernel", _fa_scaled("flash_attention_scaled_causal_kernel", True))

__all__ = ["BUNDLE_MARKER_PREFIX", "ENTRY_POINT", "KernelPattern", "forward_args", "gen_kernel", "known_patterns",
           "recognise", "register_pattern"]
