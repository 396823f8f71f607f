"""kernel-aggregate{matmul-acc=true}: fold a K-loop's `matmul` into a temporary followed by
`add(acc, acc, temporary)` into one accumulating `kernel.matmul(acc, lhs, rhs,
acc = k != k_start)` (kernel_gen/passes/kernel/kernel_aggregate.py:201-313 of the
reference, used by npu-demo-lowering with matmul_acc=True).

Conditions, checked on the IR (the fold is skipped otherwise):
  - the add follows the matmul directly, writes its first operand (`out is lhs`) and adds
    the matmul's output, which is a tile allocated in the same block and used by nothing
    else;
  - the contraction extent (lhs.shape[1] == rhs.shape[0]) is the step of exactly one
    enclosing loop, or `min(step, ...)` of it (the K loop);
  - the accumulator is defined outside that loop, is touched by nothing else inside it,
    and its last write before the loop (in the loop's block) is a zero fill.
The rewritten matmul overwrites the accumulator on the first K iteration and adds to it
afterwards, which is the sequential k order the npu_demo primitive computes
(include/npu_demo/Kernel.h:900-948): out = sum over all k, in order.
"""

from __future__ import annotations

from ..ir import Cmp, Func, Mem, Op, Sym


def _touches(op: Op, mem: Mem) -> bool:
    for inner in op.walk():
        for operand in inner.operands:
            if operand.root() is mem.root():
                return True
        if inner.result is not None and inner.result.root() is mem.root() and inner.name != "dma.alloc":
            return True
    return False


def _defined_in(block: list[Op], mem: Mem) -> bool:
    for op in block:
        for inner in op.walk():
            if inner.result is mem:
                return True
    return False


def _contraction_loop(dim: Sym, loops: list[Op]) -> Op | None:
    found = []
    for loop in loops:
        step = loop.attrs["step"]
        if dim == step or (dim.op == "min" and (dim.args[0] == step or dim.args[1] == step)):
            found.append(loop)
    return found[0] if len(found) == 1 else None


def _zero_filled_before(block: list[Op], loop: Op, acc: Mem) -> bool:
    index = next(i for i, op in enumerate(block) if op is loop)
    for op in reversed(block[:index]):
        if op.name == "dma.fill" and op.operands[0] is acc:
            return op.attrs["value"].arg is None and op.attrs["value"].value == 0.0
        if _touches(op, acc):
            return False
    return False


def kernel_aggregate(func: Func) -> int:
    """Rewrite ``func`` in place; return the number of folds."""

    folds = 0

    def visit(block: list[Op], loops: list[Op], blocks: list[list[Op]]) -> None:
        nonlocal folds
        i = 0
        while i < len(block):
            op = block[i]
            if op.name == "kernel.matmul" and op.attrs["acc"] is False and i + 1 < len(block):
                nxt = block[i + 1]
                tmp, lhs, rhs = op.operands
                if (nxt.name == "kernel.binary_elewise" and nxt.attrs["kind"] == "add" and nxt.operands[0] is nxt.operands[1]
                        and nxt.operands[2] is tmp and nxt.operands[0] is not tmp and tmp.origin == "alloc"):
                    acc = nxt.operands[0]
                    uses = [u for u in _all_ops(blocks[0]) if any(o is tmp for o in u.operands)]
                    loop = _contraction_loop(lhs.shape[1], loops) if lhs.shape[1] == rhs.shape[0] else None
                    if loop is not None and len(uses) == 2 and _defined_in(block, tmp) and acc.shape == tmp.shape:
                        body = loop.regions[0]
                        outer = blocks[loops.index(loop)]
                        others = [u for u in _all_ops(body) if u is not op and u is not nxt and u.name != "symbol.for"
                                  and u.name != "scf.if" and _touches(u, acc)]
                        if not _defined_in(body, acc) and not others and _zero_filled_before(outer, loop, acc):
                            op.operands[0] = acc
                            op.attrs["acc"] = Cmp("ne", Sym.iv(loop.attrs["iv"]), loop.attrs["start"])
                            del block[i + 1]
                            alloc_index = next(j for j, o in enumerate(block) if o.result is tmp)
                            del block[alloc_index]
                            folds += 1
                            i = max(alloc_index - 1, 0)
                            continue
            for region in op.regions:
                if op.name == "symbol.for":
                    visit(region, loops + [op], blocks + [region])
                else:
                    visit(region, loops, blocks + [region])
            i += 1

    visit(func.body, [], [func.body])
    return folds


def _all_ops(block: list[Op]):
    for op in block:
        yield from op.walk()
