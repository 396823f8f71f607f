"""Values, operations and functions of the gfx950 kernel IR.

This is the backend's reading of the reference's final IR (kernel_gen/dialect/{dma,kernel,
symbol,nn}): one function per DSL kernel whose body is a tree of operations on memory
tiles. Operation names and operand orders are the reference dialects' --

  symbol.for        iv = start .. end step step { body }          (dialect/symbol, SymbolForOp)
  scf.if            cond { then } else { else }                      (control_flow.py:112-125)
  dma.alloc         -> tile [shape] dtype space                      (operation/dma.py:134)
  dma.fill          target, value                                    (dma.py:275)
  dma.view          -> view of source at offsets/sizes/strides       (dma.py:1002)
  dma.reshape       -> source with a new (contiguous) shape          (dma.py:1046)
  dma.slice         target <- source[offsets/sizes/strides]          (dma.py:945)
  dma.deslice       target[offsets/sizes/strides] <- source          (dma.py:978)
  dma.load          target <- source[offsets/sizes/strides]          (dma.py:856)
  dma.store         target[offsets/sizes/strides] <- source          (dma.py:894)
  dma.copy          target <- source (whole tile)                    (dma.py:722)
  dma.cast          target <- source rounded to target's element type (dma.py:1119)
  dma.free          end of a tile's lifetime (no data effect)        (dma.py:198)
  arch.barrier      block-level barrier request                      (arch.py:803)
  dma.broadcast     target <- source expanded along size-1 axes      (dma.py:833)
  dma.transpose     target <- permute(source)                        (nn/transpose.py:95)
  kernel.matmul     out (+)= lhs @ rhs, acc flag / condition          (structured.py:188-218)
  kernel.img2col2d  out <- window gather of input                     (structured.py:259-305)
  kernel.exp        out <- exp(input)                                 (activation.py:108)
  kernel.reduce     out <- reduce(max|sum) over axis, keepdim         (reduction.py:152)
  kernel.binary_elewise out <- lhs (add|sub|mul|truediv|max) rhs      (binary.py:221)

-- plus one gfx950 operation, `gfx950.fused`, which the pattern pass puts in place of a
whole recognised loop nest (a call of one of the hand-written kernels of libkg_gfx950).

Memory values are SSA: every tile, view and reshape is defined once (by an argument or an
operation) and may be read and written by later operations, like the reference's memory
types (kernel_gen/dialect/nn NnMemoryType).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterator

from .sym import Sym

DTYPES = ("f32", "f16", "bf16")
ELEMENT_BYTES = {"f32": 4, "f16": 2, "bf16": 2}
TORCH_DTYPE_NAMES = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}


@dataclass(eq=False)
class Mem:
    """A memory value: an argument, a tile (dma.alloc), or a view / reshape of another."""

    name: str
    shape: tuple[Sym, ...]
    dtype: str
    space: str = "TSM"
    origin: str = "alloc"          # arg | alloc | view | reshape
    source: "Mem | None" = None    # view / reshape: the memory it aliases
    optional: bool = False         # argument that may be absent (data == NULL)

    @property
    def rank(self) -> int:
        return len(self.shape)

    def root(self) -> "Mem":
        m = self
        while m.source is not None:
            m = m.source
        return m

    def __repr__(self) -> str:
        return f"%{self.name}"


@dataclass(frozen=True)
class FVal:
    """A float operand: a literal (inf and -inf included) or a FLOAT runtime argument."""

    value: float | None = None
    arg: str | None = None

    def __str__(self) -> str:
        return self.arg if self.arg is not None else repr(self.value)


@dataclass(frozen=True)
class Present:
    """Condition: memory argument `mem` was passed (its slot's data pointer is not NULL)."""

    mem: str

    def __str__(self) -> str:
        return f"present({self.mem})"


@dataclass(frozen=True)
class Cmp:
    """Condition: a <op> b on symbolic integers; op in eq, ne, lt, le, gt, ge."""

    op: str
    a: Sym
    b: Sym

    def __str__(self) -> str:
        return f"{self.a} {self.op} {self.b}"

    def evaluate(self, env) -> bool:
        x, y = self.a.evaluate(env), self.b.evaluate(env)
        return {"eq": x == y, "ne": x != y, "lt": x < y, "le": x <= y, "gt": x > y, "ge": x >= y}[self.op]


@dataclass(frozen=True)
class Param:
    name: str
    kind: str                 # memory | int | float
    rank: int = 0
    dtype: str = "f32"
    optional: bool = False


@dataclass(eq=False)
class Op:
    name: str
    operands: list = field(default_factory=list)   # Mem values
    attrs: dict = field(default_factory=dict)
    result: Mem | None = None
    regions: list = field(default_factory=list)    # lists of Op

    def walk(self) -> Iterator["Op"]:
        yield self
        for region in self.regions:
            for op in region:
                yield from op.walk()


@dataclass(eq=False)
class Func:
    name: str
    params: list[Param]
    args: dict[str, Mem]          # memory parameters by name
    body: list[Op]

    def walk(self) -> Iterator[Op]:
        for op in self.body:
            yield from op.walk()

    def param(self, name: str) -> Param:
        for p in self.params:
            if p.name == name:
                return p
        raise KeyError(name)


def walk_block(block: list[Op]) -> Iterator[Op]:
    for op in block:
        yield from op.walk()


def parents_of(func: Func) -> dict[int, list[Op]]:
    """id(op) -> the chain of enclosing region-holding ops (outermost first)."""

    chains: dict[int, list[Op]] = {}

    def visit(block: list[Op], chain: list[Op]) -> None:
        for op in block:
            chains[id(op)] = chain
            for region in op.regions:
                visit(region, chain + [op])

    visit(func.body, [])
    return chains


# ---------------------------------------------------------------------------------------
# printing
# ---------------------------------------------------------------------------------------


def _fmt(v) -> str:
    if isinstance(v, (list, tuple)):
        return "[" + ", ".join(_fmt(x) for x in v) + "]"
    return str(v)


def format_op(op: Op, indent: int = 1) -> list[str]:
    pad = "  " * indent
    if op.name == "symbol.for":
        a = op.attrs
        lines = [f"{pad}symbol.for {a['iv']} = {a['start']} to {a['end']} step {a['step']} {{"]
        for inner in op.regions[0]:
            lines += format_op(inner, indent + 1)
        return lines + [f"{pad}}}"]
    if op.name == "scf.if":
        lines = [f"{pad}scf.if {op.attrs['cond']} {{"]
        for inner in op.regions[0]:
            lines += format_op(inner, indent + 1)
        if op.regions[1]:
            lines.append(f"{pad}}} else {{")
            for inner in op.regions[1]:
                lines += format_op(inner, indent + 1)
        return lines + [f"{pad}}}"]
    res = ""
    if op.result is not None:
        r = op.result
        res = f"%{r.name} = "
    ops = ", ".join(f"%{m.name}" for m in op.operands)
    attrs = ", ".join(f"{k}={_fmt(v)}" for k, v in op.attrs.items())
    typ = ""
    if op.result is not None:
        typ = f" : {op.result.dtype}{_fmt(op.result.shape)} {op.result.space}"
    body = f"{pad}{res}{op.name}({ops}){' {' + attrs + '}' if attrs else ''}{typ}"
    return [body]


def format_func(func: Func) -> str:
    params = []
    for p in func.params:
        if p.kind == "memory":
            params.append(f"%{p.name}: {p.dtype}[rank {p.rank}]{'?' if p.optional else ''}")
        else:
            params.append(f"%{p.name}: {p.kind}")
    lines = [f"func @{func.name}({', '.join(params)}) {{"]
    for op in func.body:
        lines += format_op(op)
    lines.append("}")
    return "\n".join(lines)
