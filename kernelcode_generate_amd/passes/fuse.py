"""kernel-pattern-fuse (gfx950): replace a recognised loop nest by one call of a
hand-written gfx950 kernel.

The three demo families lower to fixed IR shapes (after kernel-aggregate): the K-loop
matmul nest of kernel/matmul/*.py, the img2col2d -> matmul -> transpose -> add conv nest
of kernel/conv2d/*.py and the online-softmax nest of kernel/flash_attention/*.py. A nest
is recognised by what it computes, not by the kernel's name:

  1. structure: the operations, in order, with their dataflow (which tile feeds which
     operation, which argument each staged tile is read from, which tile is written back);
  2. index arithmetic: every view offset and size, loop bound and tail extent must equal
     the family's canonical expression (e.g. the lhs tile is lhs[m0 : m0 + min(tm, M - m0),
     k0 : ...]). Equality of two symbolic expressions is tested by evaluating both at
     random points of the iteration space (random shapes, runtime integers and loop
     indices drawn inside their loops) -- the identity test for polynomial-like integer
     expressions -- so any spelling of the same arithmetic matches and a different one
     does not.

A match yields a `FusedCall`: the library entry, which kernel parameter fills each of its
memory slots, and the integer / float operands (stride, dilation, pads, scale, causal) as
expressions of the kernel's parameters, evaluated by the generated entry at run time.
Anything that does not match stays on the per-operation path, which executes the IR as
written.
"""

from __future__ import annotations

import math
import random
from dataclasses import dataclass, field
from typing import Callable

from ..ir import Cmp, FVal, Func, Mem, Op, Sym, smax, smin


@dataclass(frozen=True)
class FusedCall:
    family: str                          # matmul | conv2d | flash_attention
    memory: tuple[str | None, ...]       # kernel parameter per library memory slot (None: absent)
    ints: tuple[Sym, ...] = ()           # INT slots after the memory slots
    floats: tuple[FVal, ...] = ()        # FLOAT slots (attention scale)
    trailing_ints: tuple[Sym, ...] = ()  # INT slots after the floats (attention causal flag)
    notes: tuple[str, ...] = field(default_factory=tuple)


class _NoMatch(Exception):
    pass


def _req(cond: bool, why: str = "") -> None:
    if not cond:
        raise _NoMatch(why)


# ---------------------------------------------------------------------------------------
# random evaluation of symbolic expressions over the iteration space
# ---------------------------------------------------------------------------------------


class _Space:
    """Random points of a function's iteration space: arguments and dimensions drawn at
    random, loop indices drawn inside their loops (outer loops first)."""

    def __init__(self, func: Func, loops: list[Op], seed: int = 20261202, small_dims: set | None = None) -> None:
        self.func = func
        self.loops = loops
        self.rng = random.Random(seed)
        self.small_dims = small_dims or set()

    def points(self, count: int = 48):
        made = 0
        tries = 0
        while made < count and tries < count * 50:
            tries += 1
            env: dict = {}
            for p in self.func.params:
                if p.kind == "int":
                    env[("arg", p.name)] = self.rng.randint(1, 12)
                elif p.kind == "memory":
                    for axis in range(p.rank):
                        hi = 5 if (p.name, axis) in self.small_dims else 70
                        env[("dim", p.name, axis)] = self.rng.randint(1, hi)
            ok = True
            for loop in self.loops:
                lookup = _lookup(env)
                try:
                    start = loop.attrs["start"].evaluate(lookup)
                    end = loop.attrs["end"].evaluate(lookup)
                    step = loop.attrs["step"].evaluate(lookup)
                except (KeyError, ZeroDivisionError):
                    ok = False
                    break
                if step <= 0 or end <= start:
                    ok = False
                    break
                trips = (end - start + step - 1) // step
                env[("iv", loop.attrs["iv"])] = start + step * self.rng.randrange(trips)
            if ok:
                made += 1
                yield _lookup(env)


def _lookup(env: dict) -> Callable[[Sym], int]:
    def get(s: Sym) -> int:
        if s.op == "dim":
            return env[("dim",) + tuple(s.args)]
        return env[(s.op, s.args[0])]

    return get


def _same(space: _Space, a: Sym, b: Sym) -> bool:
    seen = 0
    for point in space.points():
        try:
            if a.evaluate(point) != b.evaluate(point):
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
# structure helpers
# ---------------------------------------------------------------------------------------


def _chain(func: Func, target: Op) -> list[Op]:
    def visit(block: list[Op], chain: list[Op]):
        for op in block:
            if op is target:
                return chain
            for region in op.regions:
                found = visit(region, chain + [op])
                if found is not None:
                    return found
        return None

    found = visit(func.body, [])
    _req(found is not None)
    return found


def _block_of(func: Func, target: Op) -> list[Op]:
    chain = _chain(func, target)
    if not chain:
        return func.body
    parent = chain[-1]
    for region in parent.regions:
        if any(op is target for op in region):
            return region
    raise _NoMatch()


def _significant(block: list[Op]) -> list[Op]:
    """Operations of a block that move or compute data (allocs, views and reshapes only
    name memory)."""

    return [op for op in block if op.name not in ("dma.alloc", "dma.view", "dma.reshape")]


def _base(mem: Mem) -> Mem:
    """The tile a reshape chain names (views are kept: they select a region)."""

    while mem.origin == "reshape" and mem.source is not None:
        mem = mem.source
    return mem


def _view_of(mem: Mem) -> tuple[Mem, Op]:
    _req(mem.origin == "view" and mem.source is not None, "expected a view")
    return mem.source, mem.def_op  # type: ignore[attr-defined]


def _is_fill(op: Op, mem: Mem, value: float) -> bool:
    v = op.attrs.get("value")
    return (op.name == "dma.fill" and _base(op.operands[0]) is _base(mem) and v is not None and v.arg is None
            and (v.value == value or (math.isinf(value) and v.value == value)))


def _defs(func: Func) -> None:
    for op in func.walk():
        if op.result is not None:
            op.result.def_op = op  # type: ignore[attr-defined]


def _loads(block: list[Op]) -> dict[int, tuple[Mem, Op, Op]]:
    """tile id -> (argument, view op, deslice op) for `deslice(tile, view(arg), 0.., sizes)`
    writes in a block."""

    out = {}
    for op in block:
        if op.name == "dma.deslice":
            dst, src = op.operands
            if src.origin == "view" and src.source is not None and src.source.origin == "arg":
                out[id(_base(dst))] = (src.source, src.def_op, op)
    return out


# ---------------------------------------------------------------------------------------
# matmul
# ---------------------------------------------------------------------------------------


def _cur(iv: Sym, step: Sym, extent: Sym) -> Sym:
    return smin(step, extent - iv)


def match_matmul(func: Func) -> FusedCall:
    mms = [op for op in func.walk() if op.name == "kernel.matmul"]
    _req(len(mms) == 1, "one matmul")
    mm = mms[0]
    acc, lt, rt = mm.operands
    chain = _chain(func, mm)
    _req(len(chain) == 3 and all(op.name == "symbol.for" for op in chain), "three loops around the matmul")
    kloop = chain[-1]
    cond = mm.attrs["acc"]
    _req(isinstance(cond, Cmp) and cond.op == "ne" and cond.a == Sym.iv(kloop.attrs["iv"])
         and cond.b == kloop.attrs["start"], "K-loop accumulation")
    body = kloop.regions[0]
    sig = _significant(body)
    # k body: fills of the two tiles to 0, their loads, the matmul -- nothing else
    _req(len(sig) == 5 and sig[-1] is mm, "k-loop body")
    loads = _loads(body)
    _req(id(_base(lt)) in loads and id(_base(rt)) in loads, "staged operands")
    for op in sig[:-1]:
        if op.name == "dma.fill":
            _req(_is_fill(op, op.operands[0], 0.0) and _base(op.operands[0]) in (_base(lt), _base(rt)), "zero fill")
    a_arg, a_view, a_store = loads[id(_base(lt))]
    b_arg, b_view, b_store = loads[id(_base(rt))]
    _req(a_arg.rank == 2 and b_arg.rank == 2 and a_arg is not b_arg, "2-D operands")
    # the block around the k loop: acc zero-filled before it, optional bias, write-back
    outer = _block_of(func, kloop)
    osig = _significant(outer)
    ki = next(i for i, op in enumerate(osig) if op is kloop)
    before, after = osig[:ki], osig[ki + 1:]
    _req(any(_is_fill(op, acc, 0.0) for op in before), "acc zero fill")
    for op in before:
        _req(op.name == "dma.fill", "only fills before the k loop")
    bias = None
    if after and after[0].name == "scf.if":
        ifop = after.pop(0)
        cond = ifop.attrs["cond"]
        _req(not ifop.regions[1] and hasattr(cond, "mem"), "bias branch")
        bias = func.args[cond.mem]
        bsig = _significant(ifop.regions[0])
        _req([op.name for op in bsig][-2:] == ["dma.broadcast", "kernel.binary_elewise"], "bias add")
        add = bsig[-1]
        _req(add.attrs["kind"] == "add" and add.operands[0] is acc and add.operands[1] is acc, "acc += bias")
        bfull = add.operands[2]
        bc = bsig[-2]
        _req(bc.operands[0] is bfull, "broadcast bias")
        brow = _base(bc.operands[1])
        bloads = _loads(ifop.regions[0])
        _req(id(brow) in bloads and bloads[id(brow)][0] is bias, "bias load")
        for op in bsig[:-2]:
            _req(op.name == "dma.fill" or op is bloads[id(brow)][2], "bias staging")
        bias_view = bloads[id(brow)][1]
    _req(len(after) == 1 and after[0].name == "dma.deslice", "write-back")
    wb = after[0]
    c_arg, c_src = wb.operands
    _req(c_arg.origin == "arg" and c_arg.rank == 2 and c_arg not in (a_arg, b_arg), "output argument")
    _req(_base(c_src) is acc or (c_src.origin == "view" and c_src.source is acc), "acc written back")
    _req(func.body == [chain[0]] and _significant(chain[0].regions[0]) == [chain[1]], "perfect outer nest")
    mloop, nloop = chain[0], chain[1]
    # roles: the loop whose index offsets the lhs rows is M
    space = _Space(func, chain)
    ivs = [Sym.iv(loop.attrs["iv"]) for loop in chain]
    if not _same(space, a_view.attrs["offsets"][0], ivs[0]):
        mloop, nloop = nloop, mloop
    m0, n0, k0 = Sym.iv(mloop.attrs["iv"]), Sym.iv(nloop.attrs["iv"]), Sym.iv(kloop.attrs["iv"])
    M, K, N = Sym.dim(a_arg.name, 0), Sym.dim(a_arg.name, 1), Sym.dim(b_arg.name, 1)
    cm = _cur(m0, mloop.attrs["step"], M)
    cn = _cur(n0, nloop.attrs["step"], N)
    ck = _cur(k0, kloop.attrs["step"], K)
    zero = Sym.const(0)
    for loop, extent in ((mloop, M), (nloop, N), (kloop, K)):
        _same_all(space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    _same_all(space, a_view.attrs["offsets"] + a_view.attrs["sizes"], [m0, k0, cm, ck], "lhs tile")
    _same_all(space, b_view.attrs["offsets"] + b_view.attrs["sizes"], [k0, n0, ck, cn], "rhs tile")
    for view, store in ((a_view, a_store), (b_view, b_store)):
        _same_all(space, store.attrs["offsets"], [zero, zero], "staging offsets")
        _same_all(space, store.attrs["sizes"], view.attrs["sizes"], "staging sizes")
        _same_all(space, _base(store.operands[0]).shape, view.attrs["sizes"], "staged tile shape")
    _same_all(space, acc.shape, [cm, cn], "accumulator shape")
    _same_all(space, wb.attrs["offsets"] + wb.attrs["sizes"], [m0, n0, cm, cn], "write-back region")
    for strides in (a_view.attrs["strides"], b_view.attrs["strides"], wb.attrs["strides"]):
        _same_all(space, strides, [Sym.const(1)] * 2, "unit strides")
    if bias is not None:
        _same_all(space, bias_view.attrs["offsets"] + bias_view.attrs["sizes"], [n0, cn], "bias tile")
    return FusedCall("matmul", (c_arg.name, a_arg.name, b_arg.name, bias.name if bias is not None else None),
                     ints=(mloop.attrs["step"], nloop.attrs["step"], kloop.attrs["step"]))


# ---------------------------------------------------------------------------------------
# conv2d
# ---------------------------------------------------------------------------------------


def match_conv2d(func: Func) -> FusedCall:
    mms = [op for op in func.walk() if op.name == "kernel.matmul"]
    _req(len(mms) == 1 and mms[0].attrs["acc"] is False, "one matmul")
    mm = mms[0]
    out2, w2, col2 = mm.operands
    chain = _chain(func, mm)
    _req(len(chain) == 6 and all(op.name == "symbol.for" for op in chain), "six loops around the matmul")
    floop, nloop, hloop, wloop, iloop, cloop = chain
    _req(func.body == [floop] and all(_significant(a.regions[0]) == [b] for a, b in zip(chain[:4], chain[1:5])),
         "perfect outer nest")
    cbody = cloop.regions[0]
    sig = _significant(cbody)
    names = [op.name for op in sig]
    _req(names == ["dma.slice", "dma.slice", "kernel.img2col2d", "kernel.matmul", "dma.transpose", "dma.fill",
                   "dma.deslice", "kernel.binary_elewise"], f"conv channel-loop body {names}")
    in_slice, w_slice, i2c, _, tr, pfill, pstore, add = sig
    # dataflow
    x_arg, w_arg = in_slice.operands[1], w_slice.operands[1]
    _req(x_arg.origin == "arg" and w_arg.origin == "arg" and x_arg.rank == 4 and w_arg.rank == 4, "conv operands")
    in_tile, w_tile = in_slice.operands[0], w_slice.operands[0]
    col, src = i2c.operands
    _req(src is in_tile and _base(col2) is col and _base(w2) is w_tile, "img2col -> matmul")
    _req(tr.attrs["perm"] == (1, 0, 2, 3) and _base(tr.operands[1]) is out2, "transpose of the product")
    partial, pfull = tr.operands[0], pfill.operands[0]
    _req(_is_fill(pfill, pfull, 0.0) and pstore.operands[0] is pfull and pstore.operands[1] is partial, "partial tile")
    acc = add.operands[0]
    _req(add.attrs["kind"] == "add" and add.operands[1] is acc and add.operands[2] is pfull, "acc += partial")
    # the block around the channel loop
    ibody = iloop.regions[0]
    isig = _significant(ibody)
    ci = next(i for i, op in enumerate(isig) if op is cloop)
    before, after = isig[:ci], isig[ci + 1:]
    _req(any(_is_fill(op, acc, 0.0) for op in before) and all(op.name == "dma.fill" for op in before), "acc init")
    bias = None
    if after and after[0].name == "scf.if":
        ifop = after.pop(0)
        _req(not ifop.regions[1] and hasattr(ifop.attrs["cond"], "mem"), "bias branch")
        bias = func.args[ifop.attrs["cond"].mem]
        bsig = _significant(ifop.regions[0])
        _req([op.name for op in bsig] == ["dma.deslice", "dma.broadcast", "kernel.binary_elewise"], "bias add")
        bstore, bcast, badd = bsig
        _req(bstore.operands[1].origin == "view" and bstore.operands[1].source is bias, "bias load")
        _req(badd.attrs["kind"] == "add" and badd.operands[0] is acc and badd.operands[1] is acc
             and badd.operands[2] is bcast.operands[0], "acc += bias")
        _req(_base(bcast.operands[1]).root() is bstore.operands[0].root(), "broadcast of the bias tile")
        bias_view = bstore.operands[1].def_op
    _req(len(after) == 1 and after[0].name == "dma.deslice", "write-back")
    wb = after[0]
    y_arg, y_src = wb.operands
    _req(y_arg.origin == "arg" and y_arg.rank == 4 and y_arg not in (x_arg, w_arg), "output argument")
    _req(y_src.root() is acc.root(), "acc written back")
    # index arithmetic
    space = _Space(func, chain, small_dims={(w_arg.name, 2), (w_arg.name, 3)})
    g = i2c.attrs
    kh, kw = Sym.dim(w_arg.name, 2), Sym.dim(w_arg.name, 3)
    _same_all(space, [g["kh"], g["kw"]], [kh, kw], "kernel extents")
    sh, sw, dh, dw = g["sh"], g["sw"], g["dh"], g["dw"]
    _req(not any(e.ivs() for e in (sh, sw, dh, dw)), "loop-invariant stride and dilation")
    f0, n0, ho0, wo0, ni, c0 = (Sym.iv(loop.attrs["iv"]) for loop in chain)
    N, C, H, W = (Sym.dim(x_arg.name, i) for i in range(4))
    F = Sym.dim(w_arg.name, 0)
    Ho, Wo = hloop.attrs["end"], wloop.attrs["end"]
    _req(not Ho.ivs() and not Wo.ivs(), "output extents")
    pt = g["ph"].substitute({ho0: Sym.const(0)})
    pl = g["pl"].substitute({wo0: Sym.const(0)})
    _req(not pt.ivs() and not pl.ivs(), "pads")
    zero, one = Sym.const(0), Sym.const(1)
    for loop, extent in ((floop, F), (nloop, N), (hloop, Ho), (wloop, Wo), (cloop, C)):
        _same_all(space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    cf, cn = _cur(f0, floop.attrs["step"], F), _cur(n0, nloop.attrs["step"], N)
    cho, cwo = _cur(ho0, hloop.attrs["step"], Ho), _cur(wo0, wloop.attrs["step"], Wo)
    cc = _cur(c0, cloop.attrs["step"], C)
    _same_all(space, [iloop.attrs["start"], iloop.attrs["end"], iloop.attrs["step"]], [zero, cn, one], "image loop")
    h_org, w_org = ho0 * sh - pt, wo0 * sw - pl
    h_end = (ho0 + cho - 1) * sh - pt + (kh - 1) * dh + 1
    w_end = (wo0 + cwo - 1) * sw - pl + (kw - 1) * dw + 1
    h0, w0 = smax(h_org, 0), smax(w_org, 0)
    a = in_slice.attrs
    _same_all(space, a["offsets"], [n0 + ni, c0, h0, w0], "input window offsets")
    _same_all(space, a["sizes"], [one, cc, smin(h_end, H) - h0, smin(w_end, W) - w0], "input window sizes")
    _same_all(space, [g["ph"], g["pw"], g["pl"], g["pr"]],
              [smax(pt - ho0 * sh, 0), smax(h_end - H, 0), smax(pl - wo0 * sw, 0), smax(w_end - W, 0)], "local pads")
    _same_all(space, w_slice.attrs["offsets"] + w_slice.attrs["sizes"], [f0, c0, zero, zero, cf, cc, kh, kw], "weights")
    _same_all(space, col.shape, [one, cc, kh, kw, cho, cwo], "column tile")
    _same_all(space, pstore.attrs["offsets"] + pstore.attrs["sizes"], [zero] * 4 + [one, cf, cho, cwo], "partial")
    _same_all(space, wb.attrs["offsets"] + wb.attrs["sizes"], [n0 + ni, f0, ho0, wo0, one, cf, cho, cwo], "write-back")
    for att in (a, w_slice.attrs, wb.attrs, pstore.attrs):
        _same_all(space, att["strides"], [one] * 4, "unit strides")
    if bias is not None:
        _same_all(space, bias_view.attrs["offsets"] + bias_view.attrs["sizes"], [f0, cf], "bias tile")
    # bottom / right pads: the least that give the loops' Ho / Wo (larger ones change nothing)
    pb = smax((Ho - 1) * sh + dh * (kh - 1) + 1 - H - pt, 0)
    pr = smax((Wo - 1) * sw + dw * (kw - 1) + 1 - W - pl, 0)
    return FusedCall("conv2d", (y_arg.name, x_arg.name, w_arg.name, bias.name if bias is not None else None),
                     ints=(sh, sw, dh, dw, pt, pb, pl, pr))


# ---------------------------------------------------------------------------------------
# flash attention
# ---------------------------------------------------------------------------------------


def _uniform_fill(block: list[Op], mem: Mem) -> FVal | None:
    for op in block:
        if op.name == "dma.fill" and _base(op.operands[0]) is _base(mem):
            return op.attrs["value"]
    return None


def match_flash_attention(func: Func) -> FusedCall:
    mms = [op for op in func.walk() if op.name == "kernel.matmul"]
    _req(len(mms) == 2 and all(m.attrs["acc"] is False for m in mms), "two matmuls")
    s_mm, pv_mm = mms
    chain = _chain(func, s_mm)
    _req(len(chain) == 4 and all(op.name == "symbol.for" for op in chain) and _chain(func, pv_mm) == chain,
         "four loops around both matmuls")
    bloop, hloop, mloop, nloop = chain
    _req(func.body == [bloop] and all(_significant(a.regions[0]) == [b] for a, b in zip(chain[:2], chain[1:3])),
         "perfect outer nest")
    body = nloop.regions[0]
    sig = _significant(body)
    i = 0

    def take(name: str) -> Op:
        nonlocal i
        _req(i < len(sig) and sig[i].name == name, f"expected {name}")
        i += 1
        return sig[i - 1]

    def take_load(arg_names: set | None = None) -> tuple[Mem, Op, Op]:
        fill = take("dma.fill")
        store = take("dma.deslice")
        _req(_is_fill(fill, store.operands[0], 0.0), "zero-filled staging tile")
        src = store.operands[1]
        _req(src.origin == "view" and src.source is not None and src.source.origin == "arg" and src.source.rank == 4,
             "staging from an argument")
        return src.source, src.def_op, store

    k_arg, k_view, k_store = take_load()
    tr = take("dma.transpose")
    _req(tr.attrs["perm"] == (1, 0) and _base(tr.operands[1]) is _base(k_store.operands[0]), "K^T")
    _req(take("kernel.matmul") is s_mm, "S = Q K^T")
    score, qf, kt = s_mm.operands
    _req(kt is tr.operands[0], "S uses K^T")
    scale = None
    if sig[i].name == "kernel.binary_elewise":
        mul = take("kernel.binary_elewise")
        _req(mul.attrs["kind"] == "mul" and mul.operands[0] is score and mul.operands[1] is score, "scale")
        scale = _uniform_fill(mloop.regions[0], mul.operands[2])
        _req(scale is not None, "scale tile filled with one value")
    sfill = take("dma.fill")
    st = sfill.operands[0]
    _req(_is_fill(sfill, st, -math.inf), "-inf score tile")
    causal = False
    if sig[i].name == "symbol.for":
        rloop = take("symbol.for")
        rsig = _significant(rloop.regions[0])
        _req(len(rsig) == 1 and rsig[0].name == "dma.deslice", "row copy")
        copy = rsig[0]
        causal = True
    else:
        copy = take("dma.deslice")
    _req(copy.operands[0] is st and copy.operands[1].origin == "view" and copy.operands[1].source is score, "score copy")
    rmax = take("kernel.reduce")
    _req(rmax.attrs["kind"] == "max" and rmax.operands[1] is st, "row max")
    mx = take("kernel.binary_elewise")
    m_state = mx.operands[1]
    _req(mx.attrs["kind"] == "max" and mx.operands[2] is rmax.operands[0], "m' = max(m, rowmax)")
    m_next = mx.operands[0]
    bc1 = take("dma.broadcast")
    _req(bc1.operands[1] is m_next, "broadcast m'")
    sub = take("kernel.binary_elewise")
    _req(sub.attrs["kind"] == "sub" and sub.operands[1] is st and sub.operands[2] is bc1.operands[0], "S - m'")
    ex = take("kernel.exp")
    _req(ex.operands[1] is sub.operands[0], "P = exp(S - m')")
    p = ex.operands[0]
    rsum = take("kernel.reduce")
    _req(rsum.attrs["kind"] == "sum" and rsum.operands[1] is p, "row sum")
    osub = take("kernel.binary_elewise")
    _req(osub.attrs["kind"] == "sub" and osub.operands[1] is m_state and osub.operands[2] is m_next, "m - m'")
    oexp = take("kernel.exp")
    _req(oexp.operands[1] is osub.operands[0], "alpha = exp(m - m')")
    alpha = oexp.operands[0]
    smul = take("kernel.binary_elewise")
    l_state = smul.operands[1]
    _req(smul.attrs["kind"] == "mul" and smul.operands[2] is alpha, "l * alpha")
    sadd = take("kernel.binary_elewise")
    _req(sadd.attrs["kind"] == "add" and sadd.operands[1] is smul.operands[0] and sadd.operands[2] is rsum.operands[0],
         "l' = l alpha + rowsum")
    v_arg, v_view, v_store = take_load()
    _req(take("kernel.matmul") is pv_mm, "P V")
    part, p2, vf = pv_mm.operands
    _req(p2 is p and _base(vf) is _base(v_store.operands[0]), "P V operands")
    bc2 = take("dma.broadcast")
    _req(bc2.operands[1] is alpha, "broadcast alpha")
    wmul = take("kernel.binary_elewise")
    acc = wmul.operands[1]
    _req(wmul.attrs["kind"] == "mul" and wmul.operands[2] is bc2.operands[0], "acc * alpha")
    wadd = take("kernel.binary_elewise")
    _req(wadd.attrs["kind"] == "add" and wadd.operands[1] is wmul.operands[0] and wadd.operands[2] is part,
         "acc' = acc alpha + P V")
    for state, new in ((m_state, m_next), (l_state, sadd.operands[0]), (acc, wadd.operands[0])):
        upd = take("dma.deslice")
        _req(upd.operands[0] is state and upd.operands[1] is new, "state update")
    _req(i == len(sig), "nothing else in the key loop")
    # query block: Q staging and state init before the key loop, normalisation after it
    mblock = mloop.regions[0]
    msig = _significant(mblock)
    ni = next(j for j, op in enumerate(msig) if op is nloop)
    before, after = msig[:ni], msig[ni + 1:]
    q_loads = _loads(mblock)
    _req(id(_base(qf)) in q_loads, "Q staging")
    q_arg, q_view, q_store = q_loads[id(_base(qf))]
    inits = {id(_base(op.operands[0])): op.attrs["value"] for op in before if op.name == "dma.fill"}
    for state, value in ((m_state, -math.inf), (l_state, 0.0), (acc, 0.0)):
        v = inits.get(id(_base(state)))
        _req(v is not None and v.arg is None and v.value == value, "state initialisation")
    _req([op.name for op in after] == ["dma.broadcast", "kernel.binary_elewise", "dma.deslice"], "normalisation")
    bc3, div, wb = after
    _req(bc3.operands[1] is l_state and div.attrs["kind"] == "truediv" and div.operands[1] is acc
         and div.operands[2] is bc3.operands[0], "O = acc / l")
    o_arg, o_src = wb.operands
    _req(o_arg.origin == "arg" and o_arg.rank == 4 and o_src.root() is div.operands[0].root(), "write-back")
    args = {q_arg.name, k_arg.name, v_arg.name, o_arg.name}
    _req(len(args) == 4, "distinct q, k, v, out")
    # index arithmetic
    space = _Space(func, chain + ([rloop] if causal else []))
    b0, h0, m0, n0 = (Sym.iv(loop.attrs["iv"]) for loop in chain)
    B, H, S, D = (Sym.dim(q_arg.name, a) for a in range(4))
    br, bc = mloop.attrs["step"], nloop.attrs["step"]
    zero, one = Sym.const(0), Sym.const(1)
    cbr, cbc = _cur(m0, br, S), _cur(n0, bc, S)
    kv_end = smin(S, m0 + cbr) if causal else S
    for loop, extent in ((bloop, B), (hloop, H), (mloop, S), (nloop, kv_end)):
        _same_all(space, [loop.attrs["start"], loop.attrs["end"]], [zero, extent], "loop bounds")
    _same_all(space, [bloop.attrs["step"], hloop.attrs["step"]], [one, one], "batch and head steps")
    _same_all(space, q_view.attrs["offsets"] + q_view.attrs["sizes"], [b0, h0, m0, zero, one, one, cbr, D], "Q tile")
    for view in (k_view, v_view):
        _same_all(space, view.attrs["offsets"] + view.attrs["sizes"], [b0, h0, n0, zero, one, one, cbc, D], "K/V tile")
    for store, view, rows in ((q_store, q_view, br), (k_store, k_view, bc), (v_store, v_view, bc)):
        _same_all(space, store.attrs["offsets"], [zero] * 4, "staging offsets")
        _same_all(space, store.attrs["sizes"], view.attrs["sizes"], "staging sizes")
        _same_all(space, _base(store.operands[0]).shape, [one, one, rows, D], "staged tile")
    _same_all(space, score.shape, [br, bc], "score tile")
    cview = copy.operands[1].def_op
    if causal:
        r = Sym.iv(rloop.attrs["iv"])
        vis = smax(smin(cbc, m0 + r + 1 - n0), 0)
        _same_all(space, [rloop.attrs["start"], rloop.attrs["end"], rloop.attrs["step"]], [zero, cbr, one], "rows")
        _same_all(space, cview.attrs["offsets"] + cview.attrs["sizes"], [r, zero, one, vis], "masked row")
        _same_all(space, copy.attrs["offsets"] + copy.attrs["sizes"], [r, zero, one, vis], "masked row target")
    else:
        _same_all(space, cview.attrs["offsets"] + cview.attrs["sizes"], [zero, zero, cbr, cbc], "score region")
        _same_all(space, copy.attrs["offsets"] + copy.attrs["sizes"], [zero, zero, cbr, cbc], "score region target")
    _same_all(space, wb.attrs["offsets"] + wb.attrs["sizes"], [b0, h0, m0, zero, one, one, cbr, D], "write-back")
    if scale is None:
        scale = FVal(value=1.0)
    return FusedCall("flash_attention", (o_arg.name, q_arg.name, k_arg.name, v_arg.name), ints=(br, bc),
                     floats=(scale,), trailing_ints=(Sym.const(1 if causal else 0),),
                     notes=("causal lower-triangular mask" if causal else "no mask",))


MATCHERS = (("matmul", match_matmul), ("conv2d", match_conv2d), ("flash_attention", match_flash_attention))


def pattern_fuse(func: Func) -> FusedCall | None:
    """The fused call for ``func``'s loop nest, or None (the per-operation path)."""

    _defs(func)
    for _, matcher in MATCHERS:
        try:
            return matcher(func)
        except (_NoMatch, KeyError, IndexError, StopIteration, AttributeError):
            continue
    return None


__all__ = ["FusedCall", "MATCHERS", "match_conv2d", "match_flash_attention", "match_matmul", "pattern_fuse"]
