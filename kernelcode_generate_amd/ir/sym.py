"""Symbolic integer expressions of the gfx950 kernel IR.

The reference's DSL keeps shapes, tile sizes and loop indices as `symbol` dialect values
(kernel_gen/dialect/symbol; `symbol.for` induction variables, `min(tile, size - i)` tail
extents, kernel_gen/symbol_variable/symbol_dim.py). Here they are immutable expression
trees over five leaves -- integer constants, INT runtime arguments, dimensions of memory
arguments, loop induction variables and the launch queries of the `arch` operations
(`hw` leaves: block_id, block_num, thread_id, thread_num, subthread_id, subthread_num;
kernel_gen/operation/arch.py:652-776) -- combined with +, -, *, floor division, modulo,
min and max (Python semantics: `//` and `%` round toward negative infinity, as the DSL's
Python source means them).

An expression can be evaluated (runtime values for its leaves), rendered as C++ for the
generated entry and device code, and bounded over the iteration space of its loops
(`interval`), which is how workspace sizes of tile allocations are computed.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Mapping

_BIN = ("add", "sub", "mul", "floordiv", "mod", "min", "max")
HW_QUERIES = ("block_id", "block_num", "thread_id", "thread_num", "subthread_id", "subthread_num")


@dataclass(frozen=True)
class Sym:
    op: str                 # const | arg | dim | iv | hw | add | sub | mul | floordiv | mod | min | max
    args: tuple = ()

    # -- construction ------------------------------------------------------------------
    @staticmethod
    def const(value: int) -> "Sym":
        return Sym("const", (int(value),))

    @staticmethod
    def arg(name: str) -> "Sym":
        return Sym("arg", (name,))

    @staticmethod
    def dim(mem: str, axis: int) -> "Sym":
        return Sym("dim", (mem, int(axis)))

    @staticmethod
    def iv(name: str) -> "Sym":
        return Sym("iv", (name,))

    @staticmethod
    def hw(name: str) -> "Sym":
        if name not in HW_QUERIES:
            raise ValueError(f"unknown launch query {name!r}")
        return Sym("hw", (name,))

    @property
    def is_const(self) -> bool:
        return self.op == "const"

    @property
    def value(self) -> int:
        if self.op != "const":
            raise ValueError(f"{self} is not a constant")
        return self.args[0]

    def __add__(self, other):
        return sym_bin("add", self, other)

    def __radd__(self, other):
        return sym_bin("add", other, self)

    def __sub__(self, other):
        return sym_bin("sub", self, other)

    def __rsub__(self, other):
        return sym_bin("sub", other, self)

    def __mul__(self, other):
        return sym_bin("mul", self, other)

    def __rmul__(self, other):
        return sym_bin("mul", other, self)

    def __floordiv__(self, other):
        return sym_bin("floordiv", self, other)

    def __rfloordiv__(self, other):
        return sym_bin("floordiv", other, self)

    def __mod__(self, other):
        return sym_bin("mod", self, other)

    def __rmod__(self, other):
        return sym_bin("mod", other, self)

    def __neg__(self):
        return sym_bin("sub", 0, self)

    # -- queries -----------------------------------------------------------------------
    def leaves(self, kind: str) -> set:
        if self.op == kind:
            return {self.args[0] if kind != "dim" else self.args}
        if self.op in _BIN:
            return self.args[0].leaves(kind) | self.args[1].leaves(kind)
        return set()

    def ivs(self) -> set[str]:
        return self.leaves("iv")

    def substitute(self, mapping: Mapping["Sym", "Sym"]) -> "Sym":
        if self in mapping:
            return mapping[self]
        if self.op in _BIN:
            return sym_bin(self.op, self.args[0].substitute(mapping), self.args[1].substitute(mapping))
        return self

    def evaluate(self, env: Callable[["Sym"], int]) -> int:
        """Value with leaves (arg / dim / iv) resolved by ``env``."""

        if self.op == "const":
            return self.args[0]
        if self.op in ("arg", "dim", "iv", "hw"):
            return int(env(self))
        a = self.args[0].evaluate(env)
        b = self.args[1].evaluate(env)
        return _apply(self.op, a, b)

    def __str__(self) -> str:
        if self.op == "const":
            return str(self.args[0])
        if self.op == "arg":
            return self.args[0]
        if self.op == "dim":
            return f"{self.args[0]}.shape[{self.args[1]}]"
        if self.op == "iv":
            return self.args[0]
        if self.op == "hw":
            return f"arch.get_{self.args[0]}()"
        a, b = self.args
        if self.op in ("min", "max"):
            return f"{self.op}({a}, {b})"
        sign = {"add": "+", "sub": "-", "mul": "*", "floordiv": "//", "mod": "%"}[self.op]
        return f"({a} {sign} {b})"

    def to_c(self, leaf: Callable[["Sym"], str]) -> str:
        """C++ expression (long long); floor division and modulo through kg_floordiv / kg_mod."""

        if self.op == "const":
            return f"{self.args[0]}LL"
        if self.op in ("arg", "dim", "iv", "hw"):
            return leaf(self)
        a = self.args[0].to_c(leaf)
        b = self.args[1].to_c(leaf)
        if self.op == "add":
            return f"({a} + {b})"
        if self.op == "sub":
            return f"({a} - {b})"
        if self.op == "mul":
            return f"({a} * {b})"
        if self.op == "floordiv":
            return f"kg_floordiv({a}, {b})"
        if self.op == "mod":
            return f"kg_mod({a}, {b})"
        return f"kg_{self.op}({a}, {b})"


def _floordiv(a: int, b: int) -> int:
    if b == 0:
        raise ZeroDivisionError("symbolic floor division by zero")
    return a // b


def _apply(op: str, a: int, b: int) -> int:
    if op == "add":
        return a + b
    if op == "sub":
        return a - b
    if op == "mul":
        return a * b
    if op == "floordiv":
        return _floordiv(a, b)
    if op == "mod":
        if b == 0:
            raise ZeroDivisionError("symbolic modulo by zero")
        return a % b
    if op == "min":
        return min(a, b)
    if op == "max":
        return max(a, b)
    raise ValueError(op)


def as_sym(value) -> Sym:
    if isinstance(value, Sym):
        return value
    if isinstance(value, bool):
        raise TypeError("a bool is not a symbolic integer")
    if isinstance(value, int):
        return Sym.const(value)
    raise TypeError(f"{value!r} is not a symbolic integer")


def sym_bin(op: str, a, b) -> Sym:
    """Build ``a op b`` with constant folding and the identities x+0, x-0, x*1, x*0, x//1,
    min/max(x, x)."""

    a, b = as_sym(a), as_sym(b)
    if a.is_const and b.is_const:
        return Sym.const(_apply(op, a.value, b.value))
    if op == "add":
        if a.is_const and a.value == 0:
            return b
        if b.is_const and b.value == 0:
            return a
    elif op == "sub":
        if b.is_const and b.value == 0:
            return a
        if a == b:
            return Sym.const(0)
        # (x + c) - x and x - (x - c) style cancellations the demos produce (br - br + 1)
        if a.op == "add" and a.args[0] == b:
            return a.args[1]
        if a.op == "add" and a.args[1] == b:
            return a.args[0]
    elif op == "mul":
        if (a.is_const and a.value == 0) or (b.is_const and b.value == 0):
            return Sym.const(0)
        if a.is_const and a.value == 1:
            return b
        if b.is_const and b.value == 1:
            return a
    elif op == "floordiv":
        if b.is_const and b.value == 1:
            return a
    elif op in ("min", "max"):
        if a == b:
            return a
    return Sym(op, (a, b))


def smin(a, b) -> Sym:
    return sym_bin("min", a, b)


def smax(a, b) -> Sym:
    return sym_bin("max", a, b)


# ---------------------------------------------------------------------------------------
# bounds over an iteration space
# ---------------------------------------------------------------------------------------


def interval(expr: Sym, iv_range: Callable[[str], tuple[Sym, Sym]]) -> tuple[Sym, Sym]:
    """(lower, upper) bounds of ``expr`` with every induction variable ranging over its
    loop: ``iv_range(name)`` gives (first value, last value) as expressions of outer
    induction variables and arguments, which are bounded in turn. The result holds only
    arguments and dimensions. Division and modulo need a positive divisor (strides,
    tiles), which the front end requires of every loop step."""

    if expr.op in ("const", "arg", "dim", "hw"):
        return expr, expr
    if expr.op == "iv":
        first, last = iv_range(expr.args[0])
        lo, _ = interval(first, iv_range)
        _, hi = interval(last, iv_range)
        return lo, hi
    a_lo, a_hi = interval(expr.args[0], iv_range)
    b_lo, b_hi = interval(expr.args[1], iv_range)
    if expr.op == "add":
        return a_lo + b_lo, a_hi + b_hi
    if expr.op == "sub":
        return a_lo - b_hi, a_hi - b_lo
    if expr.op in ("min", "max"):
        f = smin if expr.op == "min" else smax
        return f(a_lo, b_lo), f(a_hi, b_hi)
    if expr.op == "mul":
        if b_lo.is_const and b_lo == b_hi and b_lo.value >= 0:
            return a_lo * b_lo, a_hi * b_lo
        if a_lo.is_const and a_lo == a_hi and a_lo.value >= 0:
            return a_lo * b_lo, a_hi * b_lo
        prods = [a_lo * b_lo, a_lo * b_hi, a_hi * b_lo, a_hi * b_hi]
        lo, hi = prods[0], prods[0]
        for p in prods[1:]:
            lo, hi = smin(lo, p), smax(hi, p)
        return lo, hi
    if expr.op == "floordiv":
        # divisor >= 1: x // d is monotone in x and moves toward 0 / -1 as d grows
        lo = smin(a_lo // b_lo, a_lo // b_hi)
        hi = smax(a_hi // b_lo, a_hi // b_hi)
        return lo, hi
    if expr.op == "mod":
        return Sym.const(0), b_hi - 1
    raise ValueError(expr.op)
