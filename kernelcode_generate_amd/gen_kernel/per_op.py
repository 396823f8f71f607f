"""Per-operation gfx950 emitter: any final IR the front end accepts -> one HIP kernel.

The reference's GPU sibling renders each final-IR operation as a call into its runtime
headers and runs the whole body on one thread of one block
(kernel_gen/dsl/gen_kernel/emit/cuda_sm89/source_bundle.py:99-151 op list, renderers
:844-1021, launch :615-620). Here:

  - the kernel's perfectly nested outer loops whose bounds do not depend on each other
    (arch-parallelize, kernel_gen/passes/arch/arch_parallelize.py:637-680, which the
    reference applies to the single top-level loop) are flattened onto the grid: a
    workgroup takes iteration `it = blockIdx.x, blockIdx.x + gridDim.x, ...` of their
    product, so any trip count runs on a bounded grid;
  - every other operation becomes a call of include/gfx950/kg_tile.h, executed by the
    workgroup's threads (kg_tile::kThreads) on strided views, with a barrier after it; loops and
    branches inside the body stay loops and branches (uniform across the workgroup);
  - every dma.alloc gets a fixed slice of the workgroup's part of a scratch workspace.
    Its size is the largest the tile can take: each dimension's maximum over the loop
    iterations it depends on, found by the generated entry by running those loops on the
    host (the dimensions of a tile rarely depend on more than one loop), with an interval
    bound when that would take more than a few million steps;
  - the entry validates every slot (kinds, ranks, dtypes, device pointers) before
    launching, allocates the workspace stream-ordered (hipMallocAsync / hipFreeAsync on
    the launch stream), and in synchronous mode reports any view that left its memory
    (the kernel skips such an operation and sets an error word) as a failed call.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from ..ir import ELEMENT_BYTES, Cmp, FVal, Func, Mem, Op, Present, Sym, interval

C_TYPES = {"f32": "float", "f16": "_Float16", "bf16": "kg_tile::Bf16"}
DTYPE_CODES = {"f32": 1, "f16": 5, "bf16": 6}
BINARY_KIND = {"add": 0, "sub": 1, "mul": 2, "truediv": 3, "max": 4}
ENUM_LIMIT = 4_000_000
MAX_GRID = 2048
SCRATCH_BYTES = 32 << 20  # cap of the allocation-free entry's scratch, per GPU (scratch_bytes)
MAX_DEVICES = 64
# largest workspace per workgroup kept in LDS (with the matmul's 32 KiB of operand stages,
# 128 of the 160 KiB a gfx950 workgroup can hold)
LDS_WORKSPACE_BYTES = 96 * 1024
QUERY_GRID = 256  # workgroups of a kernel that distributes work with arch.get_block_id / get_block_num

# Launch queries. Each workgroup is one DSL block; the operations of its body are executed
# cooperatively by the workgroup's lanes, so a block runs one DSL thread (thread and
# subthread ids are 0 and their counts 1, as on the reference's npu_demo target, whose
# thread_num is 1: kernel_gen/target/targets/npu_demo.txt).
HW_DEVICE = {"block_id": "((long long)blockIdx.x)", "block_num": "((long long)gridDim.x)", "thread_id": "0LL",
             "thread_num": "1LL", "subthread_id": "0LL", "subthread_num": "1LL"}
# On the host (workspace bounds) the block id ranges over the grid: hw_block_id is the
# enumeration variable of the bound's outermost loop.
_BLOCK_ID = Sym.hw("block_id")
_HOST_BLOCK_IV = "__hw_block_id"
HW_HOST = {"block_id": "hw_block_id", "block_num": f"{QUERY_GRID}LL", "thread_id": "0LL", "thread_num": "1LL",
           "subthread_id": "0LL", "subthread_num": "1LL"}


@dataclass
class _Plan:
    parallel: list[Op]                       # flattened outer loops, outermost first
    body: list[Op]                           # the innermost parallel loop's body (or the function's)
    allocs: list[Mem] = field(default_factory=list)
    loops: dict[str, Op] = field(default_factory=dict)       # iv -> loop
    parent: dict[str, str | None] = field(default_factory=dict)  # iv -> enclosing loop's iv


def _significant(block: list[Op]) -> list[Op]:
    return [op for op in block if op.name not in ("dma.alloc", "dma.view", "dma.reshape")]


def _syms_of(func: Func):
    for op in func.walk():
        for value in op.attrs.values():
            for x in (value if isinstance(value, (list, tuple)) else (value,)):
                if isinstance(x, Sym):
                    yield x
                elif isinstance(x, Cmp):
                    yield x.a
                    yield x.b
        for mem in op.operands + ([op.result] if op.result is not None else []):
            yield from mem.shape


def uses_block_queries(func: Func) -> bool:
    """The kernel distributes work itself with arch.get_block_id / get_block_num."""

    return any(s.leaves("hw") & {"block_id", "block_num"} for s in _syms_of(func))


def parallel_loops(func: Func) -> list[Op]:
    """arch-parallelize: the leading perfectly nested loops whose bounds use no index of
    the loops around them. A kernel that queries its block id or block count is left as
    written (the reference pass skips such functions: arch_parallelize.py:186-206)."""

    if uses_block_queries(func):
        return []
    chosen: list[Op] = []
    block = func.body
    while len(block) == 1 and block[0].name == "symbol.for":
        loop = block[0]
        outer_ivs = {l.attrs["iv"] for l in chosen}
        if any(loop.attrs[k].ivs() & outer_ivs for k in ("start", "end", "step")):
            break
        chosen.append(loop)
        block = loop.regions[0]
    return chosen


def _plan(func: Func) -> _Plan:
    par = parallel_loops(func)
    plan = _Plan(par, par[-1].regions[0] if par else func.body)

    def visit(block: list[Op], parent: str | None) -> None:
        for op in block:
            if op.name == "dma.alloc":
                plan.allocs.append(op.result)
            if op.name == "symbol.for":
                plan.loops[op.attrs["iv"]] = op
                plan.parent[op.attrs["iv"]] = parent
                visit(op.regions[0], op.attrs["iv"])
            else:
                for region in op.regions:
                    visit(region, parent)

    visit(func.body, None)
    return plan


class _Emitter:
    def __init__(self, func: Func) -> None:
        self.func = func
        self.plan = _plan(func)
        self.params = {p.name: i for i, p in enumerate(func.params)}
        self.alloc_index = {id(m): i for i, m in enumerate(self.plan.allocs)}
        self.lines: list[str] = []

    # -- expressions -----------------------------------------------------------------
    def dev_leaf(self, s: Sym) -> str:
        if s.op == "arg":
            return f"a.i_{s.args[0]}"
        if s.op == "dim":
            return f"a.s_{s.args[0]}[{s.args[1]}]"
        if s.op == "hw":
            return HW_DEVICE[s.args[0]]
        return f"iv_{s.args[0]}"

    def host_leaf(self, s: Sym) -> str:
        if s.op == "arg":
            return f"a.i_{s.args[0]}"
        if s.op == "dim":
            return f"a.s_{s.args[0]}[{s.args[1]}]"
        if s.op == "hw":
            return HW_HOST[s.args[0]]
        return f"iv_{s.args[0]}"

    def dev(self, s: Sym) -> str:
        return s.to_c(self.dev_leaf)

    def host(self, s: Sym) -> str:
        return s.to_c(self.host_leaf)

    def cond(self, c) -> str:
        if isinstance(c, bool):
            return "true" if c else "false"
        if isinstance(c, Present):
            return f"a.present_{c.mem}"
        if isinstance(c, Cmp):
            op = {"eq": "==", "ne": "!=", "lt": "<", "le": "<=", "gt": ">", "ge": ">="}[c.op]
            return f"({self.dev(c.a)} {op} {self.dev(c.b)})"
        raise ValueError(c)

    def fval(self, v: FVal) -> str:
        if v.arg is not None:
            return f"(float)a.f_{v.arg}"
        if math.isinf(v.value):
            return "__builtin_inff()" if v.value > 0 else "(-__builtin_inff())"
        return repr(float(v.value)) + "f"

    @staticmethod
    def var(m: Mem) -> str:
        return f"m_{m.name}"

    @staticmethod
    def vtype(m: Mem) -> str:
        return f"kg_tile::View<{C_TYPES[m.dtype]}, {m.rank}>"

    def arr(self, name: str, values, kind: str = "long long") -> str:
        vals = ", ".join(self.dev(v) if isinstance(v, Sym) else str(v) for v in values)
        return f"const {kind} {name}[{len(values)}] = {{{vals}}};"

    # -- body --------------------------------------------------------------------------
    def emit_block(self, block: list[Op], ind: str) -> None:
        for op in block:
            self.emit_op(op, ind)

    def emit_op(self, op: Op, ind: str) -> None:
        L = self.lines.append
        n = op.name
        err = "a.err"
        if n == "symbol.for":
            iv = op.attrs["iv"]
            L(f"{ind}{{")
            L(f"{ind}  const long long st_{iv} = {self.dev(op.attrs['step'])};")
            L(f"{ind}  const long long en_{iv} = {self.dev(op.attrs['end'])};")
            L(f"{ind}  if (st_{iv} <= 0) {{ if (threadIdx.x == 0) atomicOr({err}, 1024); }}")
            L(f"{ind}  else for (long long iv_{iv} = {self.dev(op.attrs['start'])}; iv_{iv} < en_{iv}; iv_{iv} += st_{iv}) {{")
            self.emit_block(op.regions[0], ind + "    ")
            L(f"{ind}  }}")
            L(f"{ind}}}")
            return
        if n == "scf.if":
            L(f"{ind}if ({self.cond(op.attrs['cond'])}) {{")
            self.emit_block(op.regions[0], ind + "  ")
            if op.regions[1]:
                L(f"{ind}}} else {{")
                self.emit_block(op.regions[1], ind + "  ")
            L(f"{ind}}}")
            return
        if n == "dma.alloc":
            m = op.result
            L(f"{ind}{self.arr('sh_' + m.name, m.shape)}")
            L(f"{ind}const {self.vtype(m)} {self.var(m)} = kg_tile::tile<{C_TYPES[m.dtype]}, {m.rank}>("
              f"wsb + a.ws_off[{self.alloc_index[id(m)]}], sh_{m.name});")
            return
        if n == "dma.view":
            m, (src,) = op.result, op.operands
            a = op.attrs
            L(f"{ind}{self.vtype(m)} {self.var(m)};")
            L(f"{ind}{{")
            L(f"{ind}  {self.arr('o_', a['offsets'])} {self.arr('z_', a['sizes'])} {self.arr('s_', a['strides'])}")
            L(f"{ind}  {self.var(m)} = kg_tile::subview({self.var(src)}, o_, z_, s_, {err});")
            L(f"{ind}}}")
            return
        if n == "dma.reshape":
            m, (src,) = op.result, op.operands
            L(f"{ind}{self.arr('sh_' + m.name, m.shape)}")
            L(f"{ind}const {self.vtype(m)} {self.var(m)} = kg_tile::reshape<{m.rank}>({self.var(src)}, sh_{m.name}, {err});")
            return
        if n == "dma.fill":
            L(f"{ind}kg_tile::fill({self.var(op.operands[0])}, {self.fval(op.attrs['value'])});")
            return
        if n in ("dma.deslice", "dma.slice", "dma.store", "dma.load"):
            dst, src = op.operands
            a = op.attrs
            region_of = dst if n in ("dma.deslice", "dma.store") else src
            vt = self.vtype(region_of)
            L(f"{ind}{{")
            L(f"{ind}  {self.arr('o_', a['offsets'])} {self.arr('z_', a['sizes'])} {self.arr('s_', a['strides'])}")
            L(f"{ind}  const {vt} r_ = kg_tile::subview({self.var(region_of)}, o_, z_, s_, {err});")
            if n in ("dma.deslice", "dma.store"):
                L(f"{ind}  kg_tile::copy(r_, {self.var(src)}, {err});")
            else:
                L(f"{ind}  kg_tile::copy({self.var(dst)}, r_, {err});")
            L(f"{ind}}}")
            return
        if n in ("dma.copy", "dma.cast"):
            # whole-tile copy; a cast rounds each element to the target type (to nearest even)
            L(f"{ind}kg_tile::copy({self.var(op.operands[0])}, {self.var(op.operands[1])}, {err});")
            return
        if n == "arch.barrier":
            L(f"{ind}kg_tile::sync();")
            return
        if n == "dma.free":
            L(f"{ind}// dma.free({self.var(op.operands[0])}): workspace tiles live for the whole launch")
            return
        if n == "dma.broadcast":
            L(f"{ind}kg_tile::broadcast({self.var(op.operands[0])}, {self.var(op.operands[1])}, {err});")
            return
        if n == "dma.transpose":
            L(f"{ind}{{ {self.arr('p_', op.attrs['perm'], 'int')}"
              f" kg_tile::transpose({self.var(op.operands[0])}, {self.var(op.operands[1])}, p_, {err}); }}")
            return
        if n == "kernel.matmul":
            o, l, r = op.operands
            L(f"{ind}kg_tile::matmul({self.var(o)}, {self.var(l)}, {self.var(r)}, {self.cond(op.attrs['acc'])}, {err});")
            return
        if n == "kernel.img2col2d":
            o, i = op.operands
            g = ", ".join(self.dev(op.attrs[k]) for k in ("kh", "kw", "sh", "sw", "dh", "dw", "ph", "pw", "pl", "pr"))
            L(f"{ind}kg_tile::img2col2d({self.var(o)}, {self.var(i)}, {g}, {err});")
            return
        if n == "kernel.exp":
            o, i = op.operands
            if o.rank != i.rank:
                raise ValueError("kernel.exp operands of different rank")
            L(f"{ind}kg_tile::exp({self.var(o)}, {self.var(i)}, {err});")
            return
        if n == "kernel.reduce":
            o, i = op.operands
            kind = 0 if op.attrs["kind"] == "max" else 1
            L(f"{ind}kg_tile::reduce_rows({self.var(o)}, {self.var(i)}, {kind}, {err});")
            return
        if n == "kernel.binary_elewise":
            o, l, r = op.operands
            L(f"{ind}kg_tile::binary({self.var(o)}, {self.var(l)}, {self.var(r)}, {BINARY_KIND[op.attrs['kind']]}, {err});")
            return
        raise ValueError(f"per-op emitter: unsupported operation {n}")

    # -- host-side tile bounds ----------------------------------------------------------
    def closure(self, ivs: set[str]) -> list[str]:
        """The loops to run to cover ``ivs``: those and every loop their bounds (or their
        enclosing loops' bounds) use, outermost first."""

        need = set()
        todo = list(ivs)
        while todo:
            iv = todo.pop()
            if iv in need:
                continue
            need.add(iv)
            loop = self.plan.loops[iv]
            for k in ("start", "end", "step"):
                todo.extend(loop.attrs[k].ivs())
        order = []

        def walk(block: list[Op]) -> None:
            for op in block:
                if op.name == "symbol.for":
                    if op.attrs["iv"] in need:
                        order.append(op.attrs["iv"])
                    walk(op.regions[0])
                else:
                    for region in op.regions:
                        walk(region)

        walk(self.func.body)
        return order

    def interval_ub(self, e: Sym) -> Sym:
        block = Sym.iv(_HOST_BLOCK_IV)

        def rng(iv: str):
            if iv == _HOST_BLOCK_IV:
                return Sym.const(0), Sym.const(QUERY_GRID - 1)
            loop = self.plan.loops[iv]
            return (loop.attrs["start"].substitute({_BLOCK_ID: block}),
                    (loop.attrs["end"] - 1).substitute({_BLOCK_ID: block}))

        return interval(e.substitute({_BLOCK_ID: block}), rng)[1]

    def host_bound(self, e: Sym, name: str, ind: str) -> list[str]:
        out = [f"{ind}long long {name} = 0;"]
        ivs = e.ivs()
        order = self.closure(ivs)
        per_block = "block_id" in e.leaves("hw") or any(
            "block_id" in self.plan.loops[iv].attrs[k].leaves("hw") for iv in order for k in ("start", "end", "step"))
        if not ivs and not per_block:
            return [f"{ind}long long {name} = {self.host(e)};"]
        out.append(f"{ind}{{")
        out.append(f"{ind}  long long steps = 0;")
        depth = ind + "  "
        if per_block:
            out.append(f"{depth}for (long long hw_block_id = 0; hw_block_id < {QUERY_GRID}LL; ++hw_block_id) {{")
            depth += "  "
        for iv in order:
            loop = self.plan.loops[iv]
            st = self.host(loop.attrs["step"])
            out.append(f"{depth}for (long long iv_{iv} = {self.host(loop.attrs['start'])}; "
                       f"iv_{iv} < {self.host(loop.attrs['end'])} && ({st}) > 0; iv_{iv} += {st}) {{")
            depth += "  "
        out.append(f"{depth}if (++steps > {ENUM_LIMIT}LL) {{ {name} = {self.host(self.interval_ub(e))}; goto done_{name}; }}")
        out.append(f"{depth}{name} = kg_tile::kg_max({name}, {self.host(e)});")
        for _ in range(len(order) + (1 if per_block else 0)):
            depth = depth[:-2]
            out.append(f"{depth}}}")
        out.append(f"{ind}}}")
        out.append(f"{ind}done_{name}:;")
        return out

    # -- source ------------------------------------------------------------------------
    def source(self, function: str) -> str:
        f = self.func
        L: list[str] = []
        L.append("#include <hip/hip_runtime.h>")
        L.append("#include <cstdio>")
        L.append("#include <mutex>")
        L.append('#include "kg_gfx950.h"')
        L.append('#include "gfx950/kg_generated.h"')
        L.append('#include "gfx950/kg_tile.h"')
        L.append("")
        L.append("namespace {")
        L.append("using kg_tile::kg_floordiv; using kg_tile::kg_max; using kg_tile::kg_min; using kg_tile::kg_mod;")
        L.append(f"constexpr int kMaxDevices = {MAX_DEVICES};")
        L.append(f"constexpr long long kLdsWorkspaceBytes = {LDS_WORKSPACE_BYTES};")
        L.append("")
        L.append("struct KgArgs {")
        for p in f.params:
            if p.kind == "memory":
                L.append(f"  {C_TYPES[p.dtype]}* p_{p.name}; long long s_{p.name}[{p.rank}]; long long t_{p.name}[{p.rank}];"
                         f" bool present_{p.name};")
            elif p.kind == "int":
                L.append(f"  long long i_{p.name};")
            else:
                L.append(f"  double f_{p.name};")
        L.append(f"  long long ws_off[{max(1, len(self.plan.allocs))}];")
        L.append("  long long ws_per_block;")
        L.append("  char* ws;")
        L.append("  int ws_lds;  // the workspace is the workgroup's dynamic LDS")
        L.append("  int* err;")
        L.append("};")
        L.append("")
        L.append("__global__ __launch_bounds__(kg_tile::kThreads) void kg_gfx950_generated_kernel(KgArgs a) {")
        L.append("  extern __shared__ __attribute__((aligned(16))) char kg_ws_lds[];")
        L.append("  char* wsb = a.ws_lds ? kg_ws_lds : a.ws + (long long)blockIdx.x * a.ws_per_block;")
        L.append("  (void)wsb;")
        for p in f.params:
            if p.kind == "memory":
                dims = ", ".join(f"a.s_{p.name}[{i}]" for i in range(p.rank))
                strides = ", ".join(f"a.t_{p.name}[{i}]" for i in range(p.rank))
                L.append(f"  const kg_tile::View<{C_TYPES[p.dtype]}, {p.rank}> m_{p.name}{{a.p_{p.name}, {{{dims}}}, {{{strides}}}}};")
        par = self.plan.parallel
        self.lines = []
        ind = "  "
        if par:
            for loop in par:
                iv = loop.attrs["iv"]
                L.append(f"  const long long tr_{iv} = kg_tile::kg_trips({self.dev(loop.attrs['start'])}, "
                         f"{self.dev(loop.attrs['end'])}, {self.dev(loop.attrs['step'])});")
            total = " * ".join(f"tr_{loop.attrs['iv']}" for loop in par)
            L.append(f"  const long long total = {total};")
            L.append("  for (long long it = blockIdx.x; it < total; it += gridDim.x) {")
            L.append("    long long rem = it;")
            for loop in reversed(par):
                iv = loop.attrs["iv"]
                L.append(f"    const long long iv_{iv} = {self.dev(loop.attrs['start'])} + (rem % tr_{iv}) * "
                         f"{self.dev(loop.attrs['step'])};")
                L.append(f"    rem /= tr_{iv};")
            L.append("    (void)rem;")
            ind = "    "
        elif uses_block_queries(f):
            L.append("  {  // every workgroup runs the body: the kernel distributes its work by block id")
            ind = "    "
        else:
            L.append("  if (blockIdx.x == 0) {")
            ind = "    "
        self.emit_block(self.plan.body, ind)
        L.extend(self.lines)
        L.append("  }")
        L.append("}")
        L.append("")
        L.append("__global__ void kg_gfx950_clear_word(int* w) {")
        L.append("  if (threadIdx.x == 0) *w = 0;")
        L.append("}")
        L.append("")
        L += self.entry(function)
        return "\n".join(L) + "\n"

    def scratch_bytes(self) -> int:
        """Size of the allocation-free entry's __device__ scratch. When every dma.alloc has a
        static extent the workspace per workgroup is a constant, and the scratch holds exactly
        the largest grid's slices plus the error word; kernels whose allocations depend on the
        runtime arguments get the SCRATCH_BYTES cap (a larger workspace per workgroup runs
        fewer workgroups, or fails with -3)."""

        per_block = 0
        for m in self.plan.allocs:
            count = 1
            for e in m.shape:
                if not e.is_const:
                    return SCRATCH_BYTES
                count *= max(int(e.value), 0)
            per_block += (count * ELEMENT_BYTES[m.dtype] + 255) // 256 * 256
        grid = QUERY_GRID if uses_block_queries(self.func) else MAX_GRID
        return min(SCRATCH_BYTES, per_block * grid + 256)

    def entry(self, function: str) -> list[str]:
        f = self.func
        scratch = self.scratch_bytes()
        L = ["}  // namespace", "",
             "// Scratch of kg_execute_entry_noalloc: device memory the library never allocates.",
             "// Every GPU holds its own copy until the process ends; every call on a GPU shares it",
             "// (so calls that overlap on one GPU race), and it keeps the last call's contents.",
             f"static __device__ __align__(256) char scratch[{scratch}];",
             "",
             "namespace {",
             f"constexpr long long kScratchBytes = {scratch}LL;",
             "std::mutex g_scratch_mutex;",
             "char* g_scratch[kMaxDevices] = {};",
             "",
             "// This device's address of `scratch` (looked up once per device, with it current):",
             "// the host-side name of a __device__ array is not a device address.",
             "int scratch_of_current_device(char** out) {",
             "  int dev = 0;",
             "  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {",
             "    (void)hipGetLastError();",
             f'    return kg_gfx950_fail(-2, "{function}: no current device for the scratch");',
             "  }",
             "  std::lock_guard<std::mutex> lock(g_scratch_mutex);",
             "  if (g_scratch[dev] == nullptr) {",
             "    void* p = nullptr;",
             "    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));",
             "    if (e != hipSuccess || p == nullptr) {",
             "      (void)hipGetLastError();",
             f'      return kg_gfx950_fail(-2, "{function}: hipGetSymbolAddress(scratch) failed");',
             "    }",
             "    g_scratch[dev] = static_cast<char*>(p);",
             "  }",
             "  *out = g_scratch[dev];",
             "  return 0;",
             "}",
             "",
             "int run(const KgArgSlot* s, unsigned long long n, bool no_alloc) {",
             f'  if (s == nullptr) return kg_gfx950_fail(-1, "ordered_args is null");',
             f'  if (n != {len(f.params)}ULL) return kg_gfx950_fail(-1, "{function} expects {len(f.params)} slots");',
             "  KgArgs a{};"]
        for i, p in enumerate(f.params):
            if p.kind == "memory":
                L.append(f'  if (kg_gfx950_check_memory_slot(s, {i}, {p.rank}, {1 if p.optional else 0}, '
                         f'{DTYPE_CODES[p.dtype]}, "{p.name}") != 0) return -1;')
                L.append(f"  a.present_{p.name} = s[{i}].data != nullptr;")
                L.append(f"  a.p_{p.name} = static_cast<{C_TYPES[p.dtype]}*>(s[{i}].data);")
                L.append(f"  for (int d = 0; d < {p.rank}; ++d) {{ a.s_{p.name}[d] = a.present_{p.name} ? s[{i}].shape[d] : 0; "
                         f"a.t_{p.name}[d] = a.present_{p.name} ? s[{i}].stride[d] : 0; }}")
            elif p.kind == "int":
                L.append(f'  if (s[{i}].kind != KG_ARG_INT) return kg_gfx950_fail(-1, "slot {i} ({p.name}): expected int slot");')
                L.append(f"  a.i_{p.name} = s[{i}].int_value;")
            else:
                L.append(f"  if (s[{i}].kind == KG_ARG_FLOAT) a.f_{p.name} = s[{i}].float_value;")
                L.append(f"  else if (s[{i}].kind == KG_ARG_INT) a.f_{p.name} = (double)s[{i}].int_value;")
                L.append(f'  else return kg_gfx950_fail(-1, "slot {i} ({p.name}): expected float slot");')
        # loop steps that are loop-invariant must be positive (the others are checked in the kernel)
        for iv, loop in self.plan.loops.items():
            st = loop.attrs["step"]
            if not st.ivs() and not st.is_const:
                L.append(f'  if ({self.host(st)} <= 0) return kg_gfx950_fail(-1, "{function}: loop {iv} has a non-positive step");')
        # workspace plan
        L.append("  long long off = 0;")
        for k, m in enumerate(self.plan.allocs):
            dims = []
            for d, e in enumerate(m.shape):
                name = f"ub_{k}_{d}"
                L += self.host_bound(e, name, "  ")
                dims.append(f"kg_tile::kg_max({name}, 0LL)")
            size = " * ".join(dims) if dims else "1LL"
            L.append(f"  a.ws_off[{k}] = off; off += ((({size}) * {ELEMENT_BYTES[m.dtype]}LL) + 255LL) / 256LL * 256LL;")
        L.append("  a.ws_per_block = off;")
        L += [
            "  // A workspace of at most kLdsWorkspaceBytes lives in the workgroup's LDS (private to the",
            "  // workgroup for the launch, like its slice of device memory, at a fraction of the latency);",
            "  // only the error word is then device memory. (A gfx950 workgroup holds up to 160 KiB of LDS,",
            "  // and HIP launches that much dynamic LDS without a per-function attribute.)",
            "  a.ws_lds = off > 0 && off <= kLdsWorkspaceBytes;",
            "  const long long ws_block = a.ws_lds ? 0 : off;  // device-memory workspace per workgroup",
        ]
        par = self.plan.parallel
        if par:
            trips = " * ".join(
                f"kg_tile::kg_trips({self.host(l.attrs['start'])}, {self.host(l.attrs['end'])}, {self.host(l.attrs['step'])})"
                for l in par)
            L.append(f"  const long long total = {trips};")
        elif uses_block_queries(f):
            L.append(f"  const long long total = {QUERY_GRID};  // arch.get_block_num() of the launch")
        else:
            L.append("  const long long total = 1;")
        L.append("  if (total <= 0) return kg_gfx950_finish_launch(\"" + function + "(empty)\");")
        L.append(f"  long long grid = total < {MAX_GRID} ? total : {MAX_GRID};")
        L += [
            "  hipStream_t stream = static_cast<hipStream_t>(kg_gfx950_launch_stream());",
            "  char* ws = nullptr;",
            "  if (no_alloc) {",
            "    // fewer workgroups when the scratch cannot give each its slice (the loop is block-strided)",
            "    if (ws_block > kScratchBytes - 256) {",
            "      char msg[256];",
            f'      snprintf(msg, sizeof(msg), "{function}: %lld bytes of workspace per workgroup exceed the %lld-byte '
            f'scratch of the allocation-free entry", ws_block, kScratchBytes - 256);',
            "      return kg_gfx950_fail(-3, msg);",
            "    }",
            "    const long long fit = ws_block > 0 ? (kScratchBytes - 256) / ws_block : grid;",
            ("    if (grid > fit) grid = fit;" if not uses_block_queries(f) else
             f'    if (grid > fit) return kg_gfx950_fail(-3, "{function}: the {QUERY_GRID} workgroups the kernel\'s '
             f'block queries assume do not fit the scratch of the allocation-free entry");'),
            "    if (scratch_of_current_device(&ws) != 0) return -2;",
            "  } else {",
            "    const size_t bytes = (size_t)(grid * ws_block) + 256;",
            "    if (hipMallocAsync(reinterpret_cast<void**>(&ws), bytes, stream) != hipSuccess) {",
            "      (void)hipGetLastError();",
            f'      return kg_gfx950_fail(-2, "{function}: workspace allocation failed");',
            "    }",
            "  }",
            "  a.err = reinterpret_cast<int*>(ws + grid * ws_block);",
            "  a.ws = ws;",
            "  // the error word starts at zero: cleared by a kernel (no memset node if a caller captures the stream)",
            "  hipLaunchKernelGGL(kg_gfx950_clear_word, dim3(1), dim3(64), 0, stream, a.err);",
            "  hipLaunchKernelGGL(kg_gfx950_generated_kernel, dim3((unsigned)grid), dim3(kg_tile::kThreads),",
            "                     a.ws_lds ? (unsigned)off : 0u, stream, a);",
            "  int err_word = 0;",
            "  const bool sync = kg_gfx950_launch_synchronous() != 0;",
            "  if (sync) (void)hipMemcpyAsync(&err_word, a.err, sizeof(int), hipMemcpyDeviceToHost, stream);",
            "  if (!no_alloc) (void)hipFreeAsync(ws, stream);",
            f'  const int rc = kg_gfx950_finish_launch(no_alloc ? "{function}(per-op, no-alloc)" : "{function}(per-op)");',
            "  if (rc != 0) return rc;",
            f'  if (sync && err_word != 0) return kg_gfx950_fail(-1, "{function}: an operation addressed memory '
            f'outside its view or got inconsistent shapes (error word set)");',
            "  return 0;",
            "}",
            "",
            "}  // namespace",
            "",
            'extern "C" int kg_execute_entry(const KgArgSlot* s, unsigned long long n) { return run(s, n, false); }',
            "",
            'extern "C" int kg_execute_entry_noalloc(const KgArgSlot* s, unsigned long long n) { return run(s, n, true); }',
        ]
        return L


def emit_per_op(func: Func, function: str) -> str:
    """HIP source (kernel + kg_execute_entry) executing ``func`` operation by operation."""

    return _Emitter(func).source(function)


__all__ = ["emit_per_op", "parallel_loops"]
