"""kernel-pattern-fuse (gfx950): replace a recognised loop nest by one call of a
hand-written gfx950 kernel.

A function is recognised by what it computes, not by how its source spells it:

  1. Symbolic execution. The body is run abstractly (`_Tracer`): every tile operation
     produces a value node -- a load from an argument, a fill, a region extracted or
     inserted, a reshape / transpose / broadcast, an img2col window, or a compute node
     (matmul, elementwise, exp, row reduction) -- and every write replaces the tile's
     current value. Loops become loop nodes (the value a tile carries out of the loop,
     with its initial value and its value after one body pass in terms of its value on
     entry), branches on a present memory argument become `if` nodes. Views, reshapes,
     staging copies, in-place updates and the order of independent operations therefore
     leave no trace: two programs that stage their tiles differently give the same
     compute nodes.
  2. Compute structure. The family's compute graph is looked for among the compute
     nodes (matmul accumulation over a K loop; a channel loop adding img2col-matmul
     products; the online-softmax recurrence over key blocks), commutative operands in
     either order.
  3. Element probing. Every data-movement path between the arguments and the compute
     nodes (and from the compute nodes to the stored output) is checked element by
     element: at random points of the iteration space (random shapes, runtime integers
     and loop indices drawn inside their loops, with dimensions large enough that every
     loop takes several trips) and at random elements of the tiles, the probe follows
     the movement nodes to the argument element, constant or compute-node element that
     supplies the value, and it must be the one the family's definition names (e.g. the
     lhs operand of the K-loop matmul at row i, column kk holds lhs[m0 + i, k0 + kk] for
     kk below the tail extent and zero beyond it; the img2col operand of a convolution
     holds the input pixel of the output pixel's window, or zero in the padding).

A match yields a `FusedCall`: the library entry, which kernel parameter fills each of its
memory slots, and the integer / float operands (stride, dilation, pads, scale, causal) as
expressions of the kernel's parameters, evaluated by the generated entry at run time.
Anything that does not match stays on the per-operation path, which executes the IR as
written.
"""

from __future__ import annotations

import itertools
import math
import random
from dataclasses import dataclass, field
from typing import Callable

from ..ir import Cmp, FVal, Func, Mem, Op, Present, Sym, smax, smin


@dataclass(frozen=True)
class FusedCall:
    family: str                          # matmul | conv2d | flash_attention
    memory: tuple[str | None, ...]       # kernel parameter per library memory slot (None: absent)
    ints: tuple[Sym, ...] = ()           # INT slots after the memory slots
    floats: tuple[FVal, ...] = ()        # FLOAT slots (attention scale)
    trailing_ints: tuple[Sym, ...] = ()  # INT slots after the floats (attention causal flag)
    notes: tuple[str, ...] = field(default_factory=tuple)
    tiles: tuple[Sym, ...] = ()          # the nest's tile steps (the entry's optional tile slots)


class _NoMatch(Exception):
    pass


def _req(cond: bool, why: str = "") -> None:
    if not cond:
        raise _NoMatch(why)


# ---------------------------------------------------------------------------------------
# values of the symbolic execution
# ---------------------------------------------------------------------------------------

_SERIAL = itertools.count()

# kinds whose element values are copies of other elements (or constants)
_MOVEMENT = {"fill", "arg", "undef", "extract", "insert", "reshape", "transpose", "bcast", "img2col"}
_COMMUTATIVE = {"add", "mul", "max"}


@dataclass(eq=False)
class Val:
    kind: str
    args: tuple = ()
    shape: tuple = ()
    attrs: dict = field(default_factory=dict)
    serial: int = field(default_factory=lambda: next(_SERIAL))

    def __repr__(self) -> str:
        return f"<{self.kind}#{self.serial}>"


def _zero(s: Sym) -> bool:
    return s.is_const and s.value == 0


def _one(s: Sym) -> bool:
    return s.is_const and s.value == 1


def _reshape(x: Val, shape) -> Val:
    shape = tuple(shape)
    if shape == tuple(x.shape):
        return x
    if x.kind == "reshape":
        x = x.args[0]
        if shape == tuple(x.shape):
            return x
    return Val("reshape", (x,), shape)


def _extract(x: Val, offsets, sizes, strides) -> Val:
    if all(_zero(o) for o in offsets) and all(_one(s) for s in strides) and tuple(sizes) == tuple(x.shape):
        return x
    return Val("extract", (x,), tuple(sizes), {"offsets": tuple(offsets), "strides": tuple(strides)})


def _insert(x: Val, y: Val, offsets, sizes, strides) -> Val:
    if all(_zero(o) for o in offsets) and all(_one(s) for s in strides) and tuple(sizes) == tuple(x.shape):
        return _reshape(y, x.shape)
    return Val("insert", (x, _reshape(y, sizes)), tuple(x.shape),
               {"offsets": tuple(offsets), "sizes": tuple(sizes), "strides": tuple(strides)})


@dataclass
class _Output:
    arg: Mem
    offsets: tuple
    sizes: tuple
    strides: tuple
    value: Val
    loops: tuple                 # enclosing symbol.for ops, outermost first
    conds: tuple                 # enclosing scf.if conditions


def _destination(op: Op) -> Mem | None:
    if op.name in ("dma.alloc", "dma.view", "dma.reshape", "dma.free", "arch.barrier", "symbol.for", "scf.if"):
        return None
    return op.operands[0] if op.operands else None


class _Tracer:
    """Symbolic execution of a function body over tile values."""

    def __init__(self, func: Func) -> None:
        self.func = func
        self.outputs: list[_Output] = []
        self.loops: list[Op] = []
        self.conds: list = []
        self.loop_vals: dict[int, dict[int, Val]] = {}   # id(loop op) -> {id(tile): loop value}
        self.loop_span: dict[int, tuple[int, int]] = {}  # id(loop op) -> serials created by its body
        for op in func.walk():
            if op.result is not None:
                op.result.def_op = op  # type: ignore[attr-defined]
        self.env = self.block(func.body, {})

    # -- memory access ------------------------------------------------------------------
    def read(self, m: Mem, env: dict) -> Val:
        chain = []
        x = m
        while x.source is not None:
            chain.append(x)
            x = x.source
        if x.origin == "arg":
            v = Val("arg", shape=x.shape, attrs={"mem": x})
        else:
            v = env.get(id(x))
            if v is None:
                v = Val("undef", shape=x.shape)
        for a in reversed(chain):
            if a.origin == "view":
                at = a.def_op.attrs  # type: ignore[attr-defined]
                v = _extract(v, at["offsets"], at["sizes"], at["strides"])
            else:
                v = _reshape(v, a.shape)
        return v

    def record(self, arg: Mem, offsets, sizes, strides, value: Val) -> None:
        self.outputs.append(_Output(arg, tuple(offsets), tuple(sizes), tuple(strides), value, tuple(self.loops),
                                    tuple(self.conds)))

    def write(self, m: Mem, value: Val, env: dict) -> None:
        if m.source is None:
            if m.origin == "arg":
                zero, one = Sym.const(0), Sym.const(1)
                self.record(m, [zero] * m.rank, m.shape, [one] * m.rank, _reshape(value, m.shape))
            else:
                env[id(m)] = _reshape(value, m.shape)
            return
        if m.origin == "view":
            at = m.def_op.attrs  # type: ignore[attr-defined]
            self.write_region(m.source, at["offsets"], at["sizes"], at["strides"], value, env)
        else:
            self.write(m.source, _reshape(value, m.source.shape), env)

    def write_region(self, m: Mem, offsets, sizes, strides, value: Val, env: dict) -> None:
        if m.source is None and m.origin == "arg":
            self.record(m, offsets, sizes, strides, _reshape(value, sizes))
            return
        _req(m.root().origin != "arg", "write through a view of an argument")
        self.write(m, _insert(self.read(m, env), value, offsets, sizes, strides), env)

    # -- operations -----------------------------------------------------------------------
    def block(self, ops: list[Op], env: dict) -> dict:
        for op in ops:
            self.op(op, env)
        return env

    def op(self, op: Op, env: dict) -> None:
        n, a = op.name, op.attrs
        if n == "dma.alloc":
            env[id(op.result)] = Val("undef", shape=op.result.shape)
        elif n in ("dma.view", "dma.reshape", "dma.free", "arch.barrier"):
            pass
        elif n == "dma.fill":
            t = op.operands[0]
            self.write(t, Val("fill", shape=t.shape, attrs={"value": a["value"]}), env)
        elif n in ("dma.slice", "dma.load"):
            dst, src = op.operands
            self.write(dst, _extract(self.read(src, env), a["offsets"], a["sizes"], a["strides"]), env)
        elif n in ("dma.deslice", "dma.store"):
            dst, src = op.operands
            self.write_region(dst, a["offsets"], a["sizes"], a["strides"], self.read(src, env), env)
        elif n == "dma.copy":
            dst, src = op.operands
            self.write(dst, self.read(src, env), env)
        elif n == "dma.cast":
            dst, src = op.operands
            self.write(dst, Val("cast", (self.read(src, env),), dst.shape, {"dtype": dst.dtype}), env)
        elif n == "dma.broadcast":
            dst, src = op.operands
            self.write(dst, Val("bcast", (self.read(src, env),), dst.shape), env)
        elif n == "dma.transpose":
            dst, src = op.operands
            self.write(dst, Val("transpose", (self.read(src, env),), dst.shape, {"perm": tuple(a["perm"])}), env)
        elif n == "kernel.matmul":
            o, l, r = op.operands
            if a["acc"] is False:
                v = Val("mm", (self.read(l, env), self.read(r, env)), o.shape)
            else:
                v = Val("mmacc", (self.read(o, env), self.read(l, env), self.read(r, env)), o.shape,
                        {"cond": a["acc"]})
            self.write(o, v, env)
        elif n == "kernel.binary_elewise":
            o, l, r = op.operands
            self.write(o, Val(a["kind"], (self.read(l, env), self.read(r, env)), o.shape), env)
        elif n == "kernel.exp":
            o, i = op.operands
            self.write(o, Val("exp", (self.read(i, env),), o.shape), env)
        elif n == "kernel.reduce":
            o, i = op.operands
            self.write(o, Val("r" + a["kind"], (self.read(i, env),), o.shape), env)
        elif n == "kernel.img2col2d":
            o, i = op.operands
            self.write(o, Val("img2col", (self.read(i, env),), o.shape, dict(a)), env)
        elif n == "symbol.for":
            self.loop(op, env)
        elif n == "scf.if":
            self.branch(op, env)
        else:
            raise _NoMatch(f"operation {n}")

    def loop(self, op: Op, env: dict) -> None:
        inner_allocs = {id(o.result) for o in op.walk() if o.name == "dma.alloc"}
        written: dict[int, Mem] = {}
        for o in op.walk():
            dst = _destination(o)
            if dst is not None:
                root = dst.root()
                if root.origin != "arg" and id(root) not in inner_allocs:
                    written[id(root)] = root
        ins = {}
        inner = dict(env)
        for tid, tile in written.items():
            ins[tid] = Val("in", shape=tile.shape, attrs={"tile": tile, "loop": op})
            inner[tid] = ins[tid]
        first = next(_SERIAL)
        self.loops.append(op)
        try:
            body = self.block(op.regions[0], inner)
        finally:
            self.loops.pop()
        self.loop_span[id(op)] = (first, next(_SERIAL))
        vals = {}
        for tid, tile in written.items():
            init = env.get(tid) or Val("undef", shape=tile.shape)
            vals[tid] = Val("loop", shape=tile.shape,
                            attrs={"loop": op, "tile": tile, "init": init, "body": body[tid], "in": ins[tid]})
            env[tid] = vals[tid]
        self.loop_vals[id(op)] = vals

    def branch(self, op: Op, env: dict) -> None:
        cond = op.attrs["cond"]
        results = []
        for region in op.regions:
            self.conds.append(cond)
            try:
                results.append(self.block(region, dict(env)))
            finally:
                self.conds.pop()
        then_env, else_env = results
        for tid in list(env):
            t, e = then_env.get(tid, env[tid]), else_env.get(tid, env[tid])
            if t is not env[tid] or e is not env[tid]:
                env[tid] = Val("if", shape=env[tid].shape, attrs={"cond": cond, "then": t, "else": e})


# ---------------------------------------------------------------------------------------
# random points of the iteration space
# ---------------------------------------------------------------------------------------


def _all_loops(func: Func) -> list[Op]:
    return [op for op in func.walk() if op.name == "symbol.for"]


class _Space:
    """Random points of a function's iteration space: INT arguments and memory dimensions
    drawn at random, then every loop index drawn inside its loop (outer loops first).
    Dimensions are drawn up to a bound that gives each loop with a constant step several
    trips; `seen_inner` records which loops were drawn at an index past their first
    iteration, so a match can require that every loop index was exercised."""

    def __init__(self, func: Func, seed: int = 20261202, small_dims: set | None = None) -> None:
        self.func = func
        self.loops = _all_loops(func)
        self.rng = random.Random(seed)
        self.small_dims = small_dims or set()
        steps = [l.attrs["step"].value for l in self.loops if l.attrs["step"].is_const]
        self.big = max([70] + [3 * s + 10 for s in steps])
        self.seen_inner: set[str] = set()
        self.max_trips: dict[str, int] = {}
        self.cache: list = []

    def _draw(self):
        env: dict = {}
        hi = self.rng.choice((12, 70, self.big))
        for p in self.func.params:
            if p.kind == "int":
                env[("arg", p.name)] = self.rng.randint(1, 12)
            elif p.kind == "memory":
                for axis in range(p.rank):
                    top = 5 if (p.name, axis) in self.small_dims else hi
                    env[("dim", p.name, axis)] = self.rng.randint(1, top)
        for loop in self.loops:
            look = _lookup(env)
            try:
                start = loop.attrs["start"].evaluate(look)
                end = loop.attrs["end"].evaluate(look)
                step = loop.attrs["step"].evaluate(look)
            except (KeyError, ZeroDivisionError):
                return None
            if step <= 0 or end <= start:
                return None
            trips = (end - start + step - 1) // step
            t = self.rng.randrange(trips)
            env[("iv", loop.attrs["iv"])] = start + step * t
            env[("trips", loop.attrs["iv"])] = trips
            if t > 0:
                env[("inner", loop.attrs["iv"])] = True
        return env

    def points(self, count: int = 40):
        made = 0
        for env in self.cache:
            if made >= count:
                return
            made += 1
            yield _lookup(env)
        tries = 0
        while made < count and tries < count * 60:
            tries += 1
            env = self._draw()
            if env is None:
                continue
            self.cache.append(env)
            for key, value in env.items():
                if key[0] == "inner":
                    self.seen_inner.add(key[1])
                elif key[0] == "trips":
                    self.max_trips[key[1]] = max(self.max_trips.get(key[1], 0), value)
            made += 1
            yield _lookup(env)

    def exercised(self, loops) -> bool:
        """Every loop that ever took more than one trip was also drawn past its first."""

        return all(l.attrs["iv"] in self.seen_inner or self.max_trips.get(l.attrs["iv"], 0) <= 1 for l in loops)


def _lookup(env: dict) -> Callable[[Sym], int]:
    def get(s: Sym) -> int:
        if s.op == "dim":
            return env[("dim",) + tuple(s.args)]
        return env[(s.op, s.args[0])]

    get.env = env  # type: ignore[attr-defined]
    return get


def _with_iv(pt: Callable[[Sym], int], iv: str, value: int) -> Callable[[Sym], int]:
    def get(s: Sym) -> int:
        if s.op == "iv" and s.args[0] == iv:
            return value
        return pt(s)

    return get


def _same(space: _Space, a: Sym, b: Sym) -> bool:
    seen = 0
    for pt in space.points():
        try:
            if a.evaluate(pt) != b.evaluate(pt):
                return False
        except (KeyError, ZeroDivisionError):
            return False
        seen += 1
    return seen > 0


def _same_all(space: _Space, xs, ys, why: str) -> None:
    _req(len(xs) == len(ys), why)
    for x, y in zip(xs, ys):
        _req(_same(space, x, y), why)


# ---------------------------------------------------------------------------------------
# element probes
# ---------------------------------------------------------------------------------------


class _Prober:
    """probe(v, idx, pt): where element `idx` of value `v` comes from at point `pt` --
    ("const", FVal), ("arg", name, coordinates), ("node", compute value, idx), ("undef",)
    or ("oob",) for an index outside a tile's shape."""

    def __init__(self, tracer: _Tracer) -> None:
        self.tracer = tracer
        self.movement_loop: dict[int, bool] = {}

    def shape(self, v: Val, pt) -> list[int]:
        return [d.evaluate(pt) for d in v.shape]

    def probe(self, v: Val, idx, pt, depth: int = 0):
        _req(depth < 200, "probe depth")
        idx = tuple(int(i) for i in idx)
        k = v.kind
        if k == "arg":
            # an argument element by its coordinates: the arguments' dimensions are drawn
            # independently, their agreement is the entry's run-time check
            return ("arg", v.attrs["mem"].name, idx) if len(idx) == len(v.shape) else ("oob",)
        shape = self.shape(v, pt)
        if len(idx) != len(shape) or any(i < 0 or i >= d for i, d in zip(idx, shape)):
            return ("oob",)
        if k == "fill":
            return ("const", v.attrs["value"])
        if k == "undef":
            return ("undef",)
        if k == "extract":
            off = [o.evaluate(pt) for o in v.attrs["offsets"]]
            st = [s.evaluate(pt) for s in v.attrs["strides"]]
            return self.probe(v.args[0], [o + i * s for o, i, s in zip(off, idx, st)], pt, depth + 1)
        if k == "insert":
            off = [o.evaluate(pt) for o in v.attrs["offsets"]]
            size = [s.evaluate(pt) for s in v.attrs["sizes"]]
            st = [s.evaluate(pt) for s in v.attrs["strides"]]
            inside = all(o <= i < o + z * s and (i - o) % s == 0 for o, z, s, i in zip(off, size, st, idx))
            if inside:
                return self.probe(v.args[1], [(i - o) // s for o, s, i in zip(off, st, idx)], pt, depth + 1)
            return self.probe(v.args[0], idx, pt, depth + 1)
        if k == "reshape":
            src = self.shape(v.args[0], pt)
            _req(math.prod(src) == math.prod(shape), "reshape size")
            flat = 0
            for i, d in zip(idx, shape):
                flat = flat * d + i
            out = []
            for d in reversed(src):
                out.append(flat % d)
                flat //= d
            return self.probe(v.args[0], list(reversed(out)), pt, depth + 1)
        if k == "transpose":
            perm = v.attrs["perm"]
            j = [0] * len(perm)
            for d, p in enumerate(perm):
                j[p] = idx[d]
            return self.probe(v.args[0], j, pt, depth + 1)
        if k == "bcast":
            src = self.shape(v.args[0], pt)
            lead = len(shape) - len(src)
            _req(lead >= 0, "broadcast rank")
            j = [0 if src[d] == 1 else idx[lead + d] for d in range(len(src))]
            return self.probe(v.args[0], j, pt, depth + 1)
        if k == "img2col":
            g = {key: v.attrs[key].evaluate(pt) for key in ("kh", "kw", "sh", "sw", "dh", "dw", "ph", "pw", "pl", "pr")}
            n, c, r, q, y, x = idx
            src = self.shape(v.args[0], pt)
            sy = y * g["sh"] + r * g["dh"] - g["ph"]
            sx = x * g["sw"] + q * g["dw"] - g["pl"]
            if 0 <= sy < src[2] and 0 <= sx < src[3]:
                return self.probe(v.args[0], (n, c, sy, sx), pt, depth + 1)
            return ("const", FVal(value=0.0))
        if k == "loop" and self.is_movement_loop(v):
            loop = v.attrs["loop"]
            start = loop.attrs["start"].evaluate(pt)
            end = loop.attrs["end"].evaluate(pt)
            step = loop.attrs["step"].evaluate(pt)
            _req(step > 0, "loop step")
            trips = max(0, (end - start + step - 1) // step)
            _req(trips <= 4096, "movement loop too long to probe")
            for t in reversed(range(trips)):
                got = self.probe(v.attrs["body"], idx, _with_iv(pt, loop.attrs["iv"], start + t * step), depth + 1)
                if got[0] == "node" and got[1] is v.attrs["in"]:
                    idx = got[2]
                    continue
                return got
            return self.probe(v.attrs["init"], idx, pt, depth + 1)
        return ("node", v, idx)

    def is_movement_loop(self, v: Val) -> bool:
        """A loop whose body only copies elements into the carried tile (the row mask of
        causal attention): probed by running its iterations."""

        key = v.serial
        if key not in self.movement_loop:
            lo, hi = self.tracer.loop_span[id(v.attrs["loop"])]
            ok = True
            stack, seen = [v.attrs["body"]], set()
            while stack and ok:
                x = stack.pop()
                if x.serial in seen:
                    continue
                seen.add(x.serial)
                if x.kind in _MOVEMENT:
                    stack.extend(x.args)
                elif x is v.attrs["in"] or not (lo <= x.serial < hi):
                    continue
                else:
                    ok = False
            self.movement_loop[key] = ok
        return self.movement_loop[key]


def _node(res, what: str) -> tuple[Val, tuple]:
    _req(res[0] == "node", what)
    return res[1], res[2]


def _is_const(res, value: float) -> bool:
    if res[0] != "const" or res[1].arg is not None:
        return False
    v = res[1].value
    return v == value or (math.isinf(value) and v == value)


def _operands(v: Val, kind: str) -> list[tuple[Val, Val]]:
    """The operand orders under which `v` is `kind`(a, b) (both orders when commutative)."""

    if v.kind != kind:
        return []
    a, b = v.args
    return [(a, b), (b, a)] if kind in _COMMUTATIVE else [(a, b)]


def _samples(rng: random.Random, extent: int, count: int = 3) -> list[int]:
    if extent <= 0:
        return []
    picks = {0, extent - 1}
    while len(picks) < min(extent, count + 2):
        picks.add(rng.randrange(extent))
    return sorted(picks)


class _Match:
    """Shared state of one matcher: the trace, the probe and the iteration space."""

    def __init__(self, tracer: _Tracer, small_dims: set | None = None) -> None:
        self.tracer = tracer
        self.func = tracer.func
        self.prober = _Prober(tracer)
        self.space = _Space(self.func, small_dims=small_dims)
        self.rng = random.Random(7)

    def probe(self, v: Val, idx, pt):
        return self.prober.probe(v, idx, pt)

    def single_output(self, rank: int) -> _Output:
        outs = self.tracer.outputs
        _req(len(outs) == 1, "one store into an argument")
        out = outs[0]
        _req(not out.conds and out.arg.rank == rank, "unconditional store")
        _req(all(_one(s) for s in out.strides), "unit-stride store")
        return out

    def loop_state(self, loop: Op, tile: Mem) -> Val:
        vals = self.tracer.loop_vals.get(id(loop), {})
        _req(id(tile) in vals, "loop state")
        return vals[id(tile)]

    def verify(self, check: Callable, what: str, count: int = 40, limit: int = 240) -> None:
        """Run `check` at `count` points, and at more (up to `limit`) until every loop that
        takes more than one trip has been drawn past its first."""

        loops = _all_loops(self.func)
        done = 0
        for pt in self.space.points(limit):
            check(pt)
            done += 1
            if done >= count and self.space.exercised(loops):
                return
        _req(done > 0 and self.space.exercised(loops), f"{what}: every loop index sampled past its first trip")


def _iv_of(expr: Sym, loops: tuple) -> Op:
    for loop in loops:
        if expr == Sym.iv(loop.attrs["iv"]):
            return loop
    raise _NoMatch("offset is not a loop index")


def _tail(iv: Sym, step: Sym, extent: Sym) -> Sym:
    return smin(step, extent - iv)


def _bias_split(m: "_Match", z: Val, e, pt):
    """(accumulated value, its index, bias parameter or None, bias operand, its index) for
    `z`, the value stored at an output element: either the accumulation itself or
    `if present(bias): acc + bias operand else acc`."""

    if z.kind != "if":
        return z, e, None, None, None
    cond = z.attrs["cond"]
    _req(isinstance(cond, Present), "bias branch")
    acc, ea = _node(m.probe(z.attrs["else"], e, pt), "bias-free branch")
    add, eadd = _node(m.probe(z.attrs["then"], e, pt), "bias branch")
    for x, y in _operands(add, "add"):
        if m.probe(x, eadd, pt) == ("node", acc, ea):
            return acc, ea, cond.mem, y, eadd
    raise _NoMatch("acc + bias")


# ---------------------------------------------------------------------------------------
# matmul
# ---------------------------------------------------------------------------------------


def _first_point(m: _Match):
    for pt in m.space.points(1):
        return pt
    raise _NoMatch("empty iteration space")


def _arg_read(m: _Match, v: Val, rank: int) -> str:
    """The argument an operand's elements come from (probed at its first element)."""

    for pt in m.space.points(8):
        if all(d > 0 for d in m.prober.shape(v, pt)):
            r = m.probe(v, (0,) * rank, pt)
            if r[0] == "arg":
                return r[1]
    raise _NoMatch("operand read from an argument")


def match_matmul(tracer: _Tracer) -> FusedCall:
    m = _Match(tracer)
    out = m.single_output(2)
    _req(len(out.loops) == 2, "two tile loops around the store")
    mloop, nloop = _iv_of(out.offsets[0], out.loops), _iv_of(out.offsets[1], out.loops)
    _req(mloop is not nloop, "row and column tile loops")
    # the stored value is the K-loop accumulation (+ bias)
    pt0 = _first_point(m)
    z, e = _node(m.probe(out.value, (0, 0), pt0), "stored accumulation")
    acc, _, bias, _, _ = _bias_split(m, z, e, pt0)
    _req(acc.kind == "loop" and acc.attrs["body"].kind == "mmacc", "accumulating matmul in a loop")
    body = acc.attrs["body"]
    a_op, b_op = body.args[1], body.args[2]
    kloop = acc.attrs["loop"]
    cond = body.attrs["cond"]
    _req(isinstance(cond, Cmp), "accumulation condition")
    a_arg, b_arg = _arg_read(m, a_op, 2), _arg_read(m, b_op, 2)
    _req(len({a_arg, b_arg, out.arg.name}) == 3, "distinct operands")
    _req(m.func.args[a_arg].rank == 2 and m.func.args[b_arg].rank == 2, "2-D operands")
    M, K, N = Sym.dim(a_arg, 0), Sym.dim(a_arg, 1), Sym.dim(b_arg, 1)
    m0, n0, k0 = (Sym.iv(l.attrs["iv"]) for l in (mloop, nloop, kloop))
    cm, cn = _tail(m0, mloop.attrs["step"], M), _tail(n0, nloop.attrs["step"], N)
    ck = _tail(k0, kloop.attrs["step"], K)
    zero = Sym.const(0)
    for loop, extent in ((mloop, M), (nloop, N), (kloop, K)):
        _same_all(m.space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    _same_all(m.space, list(out.sizes), [cm, cn], "stored region")

    def check(pt) -> None:
        # accumulate onto itself after the first K tile, from zero
        _req(cond.evaluate(pt) == (k0.evaluate(pt) != 0), "accumulate after the first K tile")
        vm, vn, vk = cm.evaluate(pt), cn.evaluate(pt), ck.evaluate(pt)
        i0, j0, kk0 = m0.evaluate(pt), n0.evaluate(pt), k0.evaluate(pt)
        kext = m.prober.shape(a_op, pt)[1]
        _req(m.prober.shape(b_op, pt)[0] == kext >= vk, "contraction extent")
        for i in _samples(m.rng, vm):
            for j in _samples(m.rng, vn):
                z2, e2 = _node(m.probe(out.value, (i, j), pt), "stored element")
                acc2, ea, bias2, bop, eb = _bias_split(m, z2, e2, pt)
                _req(acc2 is acc and bias2 == bias, "one accumulation")
                _req(_is_const(m.probe(acc.attrs["init"], ea, pt), 0.0), "accumulator starts at zero")
                _req(m.probe(body.args[0], ea, pt) == ("node", acc.attrs["in"], ea), "accumulates onto itself")
                if bias is not None:
                    _req(m.probe(bop, eb, pt) == ("arg", bias, (j0 + j,)), "bias element")
                for kk in _samples(m.rng, kext):
                    ra, rb = m.probe(a_op, (ea[0], kk), pt), m.probe(b_op, (kk, ea[1]), pt)
                    if kk < vk:
                        _req(ra == ("arg", a_arg, (i0 + i, kk0 + kk)), "lhs element")
                        _req(rb == ("arg", b_arg, (kk0 + kk, j0 + j)), "rhs element")
                    else:
                        _req(_is_const(ra, 0.0) or _is_const(rb, 0.0), "zero-padded K tail")

    m.verify(check, "matmul")
    steps = (mloop.attrs["step"], nloop.attrs["step"], kloop.attrs["step"])
    return FusedCall("matmul", (out.arg.name, a_arg, b_arg, bias), ints=steps, tiles=steps)


# ---------------------------------------------------------------------------------------
# conv2d
# ---------------------------------------------------------------------------------------


def _find(v: Val, kind: str) -> Val | None:
    """The first `kind` node on the movement paths into `v`."""

    stack, seen = [v], set()
    while stack:
        x = stack.pop()
        if x.serial in seen:
            continue
        seen.add(x.serial)
        if x.kind == kind:
            return x
        if x.kind in _MOVEMENT:
            stack.extend(x.args)
    return None


def match_conv2d(tracer: _Tracer) -> FusedCall:
    m = _Match(tracer)
    out = m.single_output(4)
    pt0 = _first_point(m)
    z, e = _node(m.probe(out.value, (0, 0, 0, 0), pt0), "stored accumulation")
    acc, ea0, bias, _, _ = _bias_split(m, z, e, pt0)
    _req(acc.kind == "loop", "channel accumulation loop")
    # acc' = acc + (the img2col matmul of a channel tile, possibly copied into a padded tile)
    mm = partial = None
    for x, p in _operands(acc.attrs["body"], "add"):
        if m.probe(x, ea0, pt0) == ("node", acc.attrs["in"], ea0):
            r = m.probe(p, ea0, pt0)
            if r[0] == "node" and r[1].kind == "mm":
                mm, partial = r[1], p
    _req(mm is not None, "acc += img2col matmul")
    w_op, col_op = mm.args
    i2c = _find(col_op, "img2col")
    _req(i2c is not None, "img2col operand")
    w_arg, x_arg = _arg_read(m, w_op, 2), _arg_read(m, i2c.args[0], 4)
    _req(len({w_arg, x_arg, out.arg.name}) == 3, "distinct operands")
    _req(tracer.func.args[w_arg].rank == 4 and tracer.func.args[x_arg].rank == 4, "4-D operands")
    m = _Match(tracer, small_dims={(w_arg, 2), (w_arg, 3)})
    g = i2c.attrs
    kh, kw = Sym.dim(w_arg, 2), Sym.dim(w_arg, 3)
    _same_all(m.space, [g["kh"], g["kw"]], [kh, kw], "kernel extents")
    sh, sw, dh, dw = g["sh"], g["sw"], g["dh"], g["dw"]
    _req(not any(x.ivs() for x in (sh, sw, dh, dw)), "loop-invariant stride and dilation")
    # tile loops: the store's offsets are [image, f0, ho0, wo0]
    floop, hloop, wloop = (_iv_of(out.offsets[d], out.loops) for d in (1, 2, 3))
    _req(len({id(floop), id(hloop), id(wloop)}) == 3, "distinct filter / row / column loops")
    f0, ho0, wo0 = (Sym.iv(l.attrs["iv"]) for l in (floop, hloop, wloop))
    img_loops = [l for l in out.loops if l not in (floop, hloop, wloop)]
    N, C, H, W = (Sym.dim(x_arg, i) for i in range(4))
    F = Sym.dim(w_arg, 0)
    Ho, Wo = hloop.attrs["end"], wloop.attrs["end"]
    _req(not Ho.ivs() and not Wo.ivs(), "output extents")
    pad_t = g["ph"].substitute({ho0: Sym.const(0)})
    pad_l = g["pl"].substitute({wo0: Sym.const(0)})
    _req(not pad_t.ivs() and not pad_l.ivs(), "pads")
    zero, one = Sym.const(0), Sym.const(1)
    cloop = acc.attrs["loop"]
    c0 = Sym.iv(cloop.attrs["iv"])
    for loop, extent in ((floop, F), (hloop, Ho), (wloop, Wo), (cloop, C)):
        _same_all(m.space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    cf, cho, cwo = (_tail(iv, l.attrs["step"], x) for iv, l, x in ((f0, floop, F), (ho0, hloop, Ho), (wo0, wloop, Wo)))
    cc = _tail(c0, cloop.attrs["step"], C)
    _same_all(m.space, list(out.sizes), [one, cf, cho, cwo], "stored region")
    # images: one loop over [0, N), or batch tiles with an image loop inside
    img = out.offsets[0]
    if len(img_loops) == 1:
        (nl,) = img_loops
        _same_all(m.space, [nl.attrs["start"], nl.attrs["end"], nl.attrs["step"], img],
                  [zero, N, one, Sym.iv(nl.attrs["iv"])], "image loop")
    else:
        _req(len(img_loops) == 2, "image loops")
        outer, inner = img_loops
        n0, ni = Sym.iv(outer.attrs["iv"]), Sym.iv(inner.attrs["iv"])
        _same_all(m.space, [outer.attrs["start"], outer.attrs["end"]], [zero, N], "batch tile loop")
        _same_all(m.space, [inner.attrs["end"] - inner.attrs["start"], inner.attrs["step"], img],
                  [_tail(n0, outer.attrs["step"], N), one, n0 + (ni - inner.attrs["start"])], "image loop")

    def check(pt) -> None:
        vf, vh, vw, vc = (x.evaluate(pt) for x in (cf, cho, cwo, cc))
        vkh, vkw = kh.evaluate(pt), kw.evaluate(pt)
        n_img, fb, hb, wb, cb = (x.evaluate(pt) for x in (img, f0, ho0, wo0, c0))
        s_h, s_w, d_h, d_w = (x.evaluate(pt) for x in (sh, sw, dh, dw))
        p_t, p_l = pad_t.evaluate(pt), pad_l.evaluate(pt)
        vH, vW = H.evaluate(pt), W.evaluate(pt)
        kext = m.prober.shape(w_op, pt)[1]
        _req(m.prober.shape(col_op, pt)[0] == kext >= vc * vkh * vkw, "contraction extent")
        for f in _samples(m.rng, vf, 2):
            for y in _samples(m.rng, vh, 2):
                for x in _samples(m.rng, vw, 2):
                    z2, e2 = _node(m.probe(out.value, (0, f, y, x), pt), "stored element")
                    acc2, ea, bias2, bop, eb = _bias_split(m, z2, e2, pt)
                    _req(acc2 is acc and bias2 == bias, "one accumulation")
                    _req(_is_const(m.probe(acc.attrs["init"], ea, pt), 0.0), "accumulator starts at zero")
                    if bias is not None:
                        _req(m.probe(bop, eb, pt) == ("arg", bias, (fb + f,)), "bias element")
                    mm2, (fi, pi) = _node(m.probe(partial, ea, pt), "channel-tile product")
                    _req(mm2 is mm, "one product")
                    for k in _samples(m.rng, kext, 4):
                        rw, rc = m.probe(w_op, (fi, k), pt), m.probe(col_op, (k, pi), pt)
                        if k >= vc * vkh * vkw:
                            _req(_is_const(rw, 0.0) or _is_const(rc, 0.0), "zero-padded channel tail")
                            continue
                        c, rem = divmod(k, vkh * vkw)
                        r, q = divmod(rem, vkw)
                        _req(rw == ("arg", w_arg, (fb + f, cb + c, r, q)), "weight element")
                        hh = (hb + y) * s_h + r * d_h - p_t
                        ww = (wb + x) * s_w + q * d_w - p_l
                        if 0 <= hh < vH and 0 <= ww < vW:
                            _req(rc == ("arg", x_arg, (n_img, cb + c, hh, ww)), "input element")
                        else:
                            _req(_is_const(rc, 0.0), "padding element")

    m.verify(check, "conv2d")
    # bottom / right pads: the least that give the loops' Ho / Wo (larger ones change nothing)
    pad_b = smax((Ho - 1) * sh + dh * (kh - 1) + 1 - H - pad_t, 0)
    pad_r = smax((Wo - 1) * sw + dw * (kw - 1) + 1 - W - pad_l, 0)
    tile_n = img_loops[0].attrs["step"] if len(img_loops) == 2 else one
    return FusedCall("conv2d", (out.arg.name, x_arg, w_arg, bias), ints=(sh, sw, dh, dw, pad_t, pad_b, pad_l, pad_r),
                     tiles=(floop.attrs["step"], cloop.attrs["step"], tile_n, hloop.attrs["step"], wloop.attrs["step"]))


# ---------------------------------------------------------------------------------------
# flash attention
# ---------------------------------------------------------------------------------------


def _uniform_fill(m: _Match, v: Val, pt) -> FVal | None:
    """The value every element of `v` holds when it is one filled constant."""

    got = None
    for e in itertools.product(*[_samples(m.rng, d, 2) for d in m.prober.shape(v, pt)]):
        r = m.probe(v, e, pt)
        if r[0] != "const" or (got is not None and r[1] != got):
            return None
        got = r[1]
    return got


def match_flash_attention(tracer: _Tracer) -> FusedCall:
    m = _Match(tracer)
    out = m.single_output(4)
    _req(len(out.loops) == 3, "batch, head and query-block loops")
    bloop, hloop, qloop = (_iv_of(out.offsets[d], out.loops) for d in range(3))
    _req(_zero(out.offsets[3]), "whole rows stored")
    pt0 = _first_point(m)
    # O = acc / broadcast(l), both carried out of the key loop
    div, e = _node(m.probe(out.value, (0, 0, 0, 0), pt0), "normalised output")
    _req(div.kind == "truediv", "O = acc / l")
    lacc, ea = _node(m.probe(div.args[0], e, pt0), "accumulator")
    lsum, el = _node(m.probe(div.args[1], e, pt0), "row sum")
    _req(lacc.kind == "loop" and lsum.kind == "loop" and lacc.attrs["loop"] is lsum.attrs["loop"], "key loop states")
    kloop = lacc.attrs["loop"]
    acc_in, sum_in = lacc.attrs["in"], lsum.attrs["in"]
    # acc' = acc * broadcast(alpha) + P @ V
    found = None
    for scaled, pv_path in _operands(lacc.attrs["body"], "add"):
        r1, rpv = m.probe(scaled, ea, pt0), m.probe(pv_path, ea, pt0)
        if r1[0] != "node" or rpv[0] != "node" or rpv[1].kind != "mm":
            continue
        for y, alpha_b in _operands(r1[1], "mul"):
            ral = m.probe(alpha_b, r1[2], pt0)
            if m.probe(y, r1[2], pt0) == ("node", acc_in, ea) and ral[0] == "node" and ral[1].kind == "exp":
                found = (scaled, r1[1], alpha_b, pv_path, rpv[1], ral[1])
    _req(found is not None, "acc * alpha + P V")
    scaled_acc, mul_acc, alpha_b, pv_path, pv, alpha = found
    p, v_op = pv.args
    _req(p.kind == "exp" and p.args[0].kind == "sub", "P = exp(S - m')")
    s_masked, m_b = p.args[0].args
    # alpha = exp(m - m'), m' = max(m, rowmax(S))
    _req(alpha.args[0].kind == "sub", "alpha = exp(m - m')")
    m_path, mnew_path = alpha.args[0].args
    m_in, _ = _node(m.probe(m_path, (0, 0), pt0), "running max")
    _req(m_in.kind == "in" and m_in.attrs["loop"] is kloop, "running max state")
    mnew, _ = _node(m.probe(mnew_path, (0, 0), pt0), "m'")
    rowmax = None
    for x, y in _operands(mnew, "max"):
        ry = m.probe(y, (0, 0), pt0)
        if m.probe(x, (0, 0), pt0) == ("node", m_in, (0, 0)) and ry[0] == "node" and ry[1].kind == "rmax":
            rowmax = ry[1]
    _req(rowmax is not None and rowmax.args[0] is s_masked, "m' = max(m, rowmax(S)) over the scores P reads")
    lmax = m.loop_state(kloop, m_in.attrs["tile"])
    # l' = l * alpha + rowsum(P)
    lsum_parts = None
    for x, rs in _operands(lsum.attrs["body"], "add"):
        rx, rr = m.probe(x, el, pt0), m.probe(rs, el, pt0)
        if rx[0] == "node" and rr[0] == "node" and rr[1].kind == "rsum" and rr[1].args[0] is p:
            for y, a2 in _operands(rx[1], "mul"):
                if m.probe(y, rx[2], pt0) == ("node", sum_in, el) and m.probe(a2, rx[2], pt0)[:2] == ("node", alpha):
                    lsum_parts = (x, a2, rs, rr[1])
    _req(lsum_parts is not None, "l' = l alpha + rowsum(P)")
    lsum_x, lsum_a, lsum_rs, rowsum = lsum_parts
    # S = Q K^T, optionally times a uniform scale; the masked copy P and the row max read
    s_src = None
    for pt in m.space.points(12):
        r = m.probe(s_masked, (0, 0), pt)
        if r[0] == "node":
            s_src = r[1]
            break
    _req(s_src is not None, "scores")
    scale, scale_tile = FVal(value=1.0), None
    s_mm = s_src
    if s_src.kind == "mul":
        s_mm = None
        for x, sc in _operands(s_src, "mul"):
            u = _uniform_fill(m, sc, pt0)
            if x.kind == "mm" and u is not None:
                s_mm, scale, scale_tile = x, u, sc
        _req(s_mm is not None, "uniform scale")
    _req(s_mm.kind == "mm", "S = Q K^T")
    q_op, k_op = s_mm.args
    qa, ka, va = _arg_read(m, q_op, 2), _arg_read(m, k_op, 2), _arg_read(m, v_op, 2)
    _req(len({qa, ka, va, out.arg.name}) == 4, "distinct q, k, v, out")
    _req(all(m.func.args[a].rank == 4 for a in (qa, ka, va)), "4-D q, k, v")
    B, Hh, S, D = (Sym.dim(qa, a) for a in range(4))
    b0, h0, q0, n0 = (Sym.iv(l.attrs["iv"]) for l in (bloop, hloop, qloop, kloop))
    br, bc = qloop.attrs["step"], kloop.attrs["step"]
    zero, one = Sym.const(0), Sym.const(1)
    cbr, cbc = _tail(q0, br, S), _tail(n0, bc, S)
    for loop, extent in ((bloop, B), (hloop, Hh), (qloop, S)):
        _same_all(m.space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    _same_all(m.space, [bloop.attrs["step"], hloop.attrs["step"], kloop.attrs["start"]], [one, one, zero], "loops")
    _same_all(m.space, list(out.sizes), [one, one, cbr, D], "stored rows")
    full_kv = _same(m.space, kloop.attrs["end"], S)
    _req(full_kv or _same(m.space, kloop.attrs["end"], smin(S, q0 + cbr)), "key loop end")
    seen = {"causal": None}

    def check(pt) -> None:
        vb, vh, vq, vn = (x.evaluate(pt) for x in (b0, h0, q0, n0))
        rows, cols, dd = cbr.evaluate(pt), cbc.evaluate(pt), D.evaluate(pt)
        srows, scols = m.prober.shape(s_masked, pt)
        _req(srows >= rows and scols >= cols, "score tile")
        _req(m.prober.shape(q_op, pt)[1] == dd and m.prober.shape(k_op, pt)[0] == dd, "head dimension")
        vrows, vcols = m.prober.shape(v_op, pt)
        _req(vrows == scols and vcols >= dd, "V tile")
        for i in _samples(m.rng, rows, 2):
            row = (i, 0)
            for d in _samples(m.rng, dd, 2):
                # stored element -> acc[i, d] / l[i]
                z, e2 = _node(m.probe(out.value, (0, 0, i, d), pt), "stored element")
                _req(z is div, "one normalisation")
                ia = m.probe(div.args[0], e2, pt)
                _req(ia[:2] == ("node", lacc) and ia[2][0] == i, "acc of the row")
                ia = ia[2]
                _req(m.probe(div.args[1], e2, pt) == ("node", lsum, row), "l of the row")
                _req(_is_const(m.probe(lacc.attrs["init"], ia, pt), 0.0), "acc starts at zero")
                r1 = m.probe(scaled_acc, ia, pt)
                _req(r1[:2] == ("node", mul_acc), "acc * alpha")
                _req(m.probe(y_of(mul_acc, alpha_b), r1[2], pt) == ("node", acc_in, ia), "acc of the row")
                _req(m.probe(alpha_b, r1[2], pt) == ("node", alpha, row), "alpha of the row")
                _req(m.probe(pv_path, ia, pt) == ("node", pv, ia), "P V element")
                for j in _samples(m.rng, scols, 3):
                    rv = m.probe(v_op, (j, d), pt)
                    if j < cols:
                        _req(rv == ("arg", va, (vb, vh, vn + j, d)), "V element")
                    else:
                        _req(rv[0] == "const" and rv[1].arg is None and math.isfinite(rv[1].value), "finite V pad")
            _req(_is_const(m.probe(lsum.attrs["init"], row, pt), 0.0), "l starts at zero")
            _req(_is_const(m.probe(lmax.attrs["init"], row, pt), -math.inf), "m starts at -inf")
            _req(m.probe(lmax.attrs["body"], row, pt) == ("node", mnew, row), "m <- m'")
            _req(m.probe(mnew_path, row, pt) == ("node", mnew, row), "m' of the row")
            _req(m.probe(m_path, row, pt) == ("node", m_in, row), "m of the row")
            rx = m.probe(lsum_x, row, pt)
            _req(rx[0] == "node" and m.probe(lsum_a, rx[2], pt) == ("node", alpha, row), "l * alpha of the row")
            _req(m.probe(lsum_rs, row, pt) == ("node", rowsum, row), "rowsum of the row")
            for j in _samples(m.rng, scols, 4):
                _req(m.probe(m_b, (i, j), pt) == ("node", mnew, row), "broadcast m'")
                rs = m.probe(s_masked, (i, j), pt)
                hidden = j >= cols
                if not hidden and vn + j > vq + i:
                    # a key after the query: masked exactly when the program is causal
                    if seen["causal"] is None:
                        seen["causal"] = _is_const(rs, -math.inf)
                    hidden = seen["causal"]
                if hidden:
                    _req(_is_const(rs, -math.inf), "masked score")
                    continue
                _req(rs == ("node", s_src, (i, j)), "score element")
                if scale_tile is not None:
                    _req(m.probe(scale_tile, (i, j), pt) == ("const", scale), "scale element")
                for d in _samples(m.rng, dd, 2):
                    _req(m.probe(q_op, (i, d), pt) == ("arg", qa, (vb, vh, vq + i, d)), "Q element")
                    _req(m.probe(k_op, (d, j), pt) == ("arg", ka, (vb, vh, vn + j, d)), "K element")

    def y_of(mul: Val, alpha_operand: Val) -> Val:
        a, b = mul.args
        return b if a is alpha_operand else a

    m.verify(check, "flash attention")
    causal = seen["causal"]
    _req(full_kv or causal is True, "keys past the query block are skipped only under a causal mask")
    return FusedCall("flash_attention", (out.arg.name, qa, ka, va), ints=(br, bc), floats=(scale,),
                     trailing_ints=(Sym.const(1 if causal else 0),),
                     notes=("causal lower-triangular mask" if causal else "no mask",), tiles=(br, bc))


MATCHERS = (("matmul", match_matmul), ("conv2d", match_conv2d), ("flash_attention", match_flash_attention))


def pattern_fuse(func: Func) -> FusedCall | None:
    """The fused call for ``func``'s loop nest, or None (the per-operation path)."""

    try:
        tracer = _Tracer(func)
    except (_NoMatch, KeyError, IndexError, AttributeError):
        return None
    for _, matcher in MATCHERS:
        try:
            return matcher(tracer)
        except (_NoMatch, KeyError, IndexError, StopIteration, AttributeError, ZeroDivisionError, ValueError):
            continue
    return None


__all__ = ["FusedCall", "MATCHERS", "match_conv2d", "match_flash_attention", "match_matmul", "pattern_fuse"]
