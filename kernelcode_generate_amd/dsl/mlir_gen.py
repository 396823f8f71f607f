"""DSL front end: a kernel's Python source -> gfx950 kernel IR.

The reference parses the DSL function's AST into xDSL IR (`mlir_gen(fn, *args)`,
kernel_gen/dsl/ast/mlir_gen.py:66-95). This front end does the same walk over Python's
`ast` without xDSL: it interprets the function body abstractly, with

  - memory parameters as IR memory values whose shapes are symbolic dimensions of the
    runtime arguments (`lhs.get_shape()[0]` is `lhs.shape[0]`), INT parameters as
    symbolic arguments and FLOAT parameters as float operands;
  - module constants (tile sizes, strides, pads of the static demos) read from the
    function's globals, so they enter the IR as integer constants;
  - `for i in loop(start, end, step)` as a `symbol.for` region (the body is walked once,
    with `i` a symbolic induction variable), `if x is not None` on a memory parameter as
    an `scf.if present(x)`, `if a == b` on symbols as an `scf.if` on the comparison, and
    any test on plain Python values decided while walking;
  - `min` / `max` and integer arithmetic on symbols as symbolic expressions;
  - each DSL operation call (kernel_gen.operation's `dma.*`, `kernel.*`, `nn.transpose`;
    here kernelcode_generate_amd.operation) as the IR operation of the same name; the
    operations that return a new tile (`slice`, `load`, `copy`, `cast`, `transpose`) as an
    allocation followed by the target-first operation, as the reference's lowering bridges
    them (kernel_gen/operation/dma.py:945-975); `flatten` as a reshape;
  - the `arch` launch queries (`get_block_id()` ...) as symbolic launch values.

Runtime arguments decide parameter kinds, as they do for the reference's mlir_gen: a tensor
or array is a memory parameter (its rank and element type are taken from it), None an
absent memory parameter (rank from the `Tensor[...]` annotation), an int an INT and a
float a FLOAT parameter.
"""

from __future__ import annotations

import ast
import builtins
import inspect
import math
import textwrap
import types
from dataclasses import dataclass, replace
from enum import Enum
from numbers import Integral, Real
from typing import Any, Callable, Sequence

from ..core.error import ErrorKind, ErrorModule, KernelCodeError
from ..ir import TORCH_DTYPE_NAMES, Cmp, FVal, Func, Mem, Op, Param, Present, Sym, as_sym, smax, smin, sym_bin
from ..ir.sym import HW_QUERIES
from ..operation.kernel import KernelBinaryElewiseKind, KernelReduceKind
from ..symbol_variable import MemorySpace, NumericType


def _error(message: str, node: ast.AST | None = None) -> KernelCodeError:
    where = f" (line {node.lineno})" if node is not None and hasattr(node, "lineno") else ""
    return KernelCodeError(ErrorKind.CONTRACT, ErrorModule.KERNEL, f"mlir_gen: {message}{where}")


@dataclass
class _Method:
    name: str
    mem: Mem


def _dtype_of(value: Any) -> str:
    name = str(getattr(value, "dtype", "")).replace("torch.", "")
    if name not in TORCH_DTYPE_NAMES:
        raise _error(f"unsupported memory dtype {name!r} (f32, f16 and bf16 are)")
    return TORCH_DTYPE_NAMES[name]


def _is_memory(value: Any) -> bool:
    return hasattr(value, "shape") and hasattr(value, "dtype") and not isinstance(value, (Integral, Real))


def _annotation_rank(annotation: ast.expr | None) -> int | None:
    """Rank of a `"Tensor[f32, A, B]"` annotation (string or subscript form)."""

    if annotation is None:
        return None
    text = annotation.value if isinstance(annotation, ast.Constant) and isinstance(annotation.value, str) else \
        ast.unparse(annotation)
    text = text.strip()
    if not text.startswith("Tensor[") or not text.endswith("]"):
        return None
    parts = [p.strip() for p in text[len("Tensor["):-1].split(",")]
    return len(parts) - 1


def _space(value: Any) -> str:
    if isinstance(value, MemorySpace):
        return value.value
    if isinstance(value, Enum) and type(value).__name__ == "MemorySpace":
        return str(value.name)
    raise _error(f"memory space expected, got {value!r}")


def _element(value: Any) -> str:
    if isinstance(value, NumericType):
        return value.value
    if isinstance(value, Enum) and type(value).__name__ == "NumericType":
        return {"Float32": "f32", "Float16": "f16", "BFloat16": "bf16"}.get(value.name, "f32")
    raise _error(f"element type expected, got {value!r}")


_BINARY_KINDS = {"kernel.add": "add", "kernel.sub": "sub", "kernel.mul": "mul", "kernel.truediv": "truediv",
                 "kernel.max": "max"}


class _Builder:
    def __init__(self, fdef: ast.FunctionDef, globals_: dict, free: dict, runtime_args: Sequence[Any]) -> None:
        self.globals = globals_
        self.fdef = fdef
        self.scopes: list[dict[str, Any]] = [dict(free)]
        self.depth = 0
        self.block: list[Op] = []
        self.counter = 0
        self.names: set[str] = set()
        self.params: list[Param] = []
        self.args: dict[str, Mem] = {}
        self._bind_params(runtime_args)

    @classmethod
    def of_function(cls, func_obj: Callable, runtime_args: Sequence[Any]) -> "_Builder":
        try:
            source = textwrap.dedent(inspect.getsource(func_obj))
        except (OSError, TypeError):
            raise _error(f"{func_obj!r} is not a Python function with source") from None
        fdefs = [n for n in ast.parse(source).body if isinstance(n, ast.FunctionDef)]
        if not fdefs:
            raise _error(f"{func_obj!r} is not a Python function with source")
        # free variables of a kernel defined inside another function are visible too
        cells = getattr(func_obj, "__closure__", None) or ()
        free = dict(zip(func_obj.__code__.co_freevars, (c.cell_contents for c in cells)))
        return cls(fdefs[0], getattr(func_obj, "__globals__", {}), free, runtime_args)

    # -- names -------------------------------------------------------------------------
    def fresh(self, hint: str) -> str:
        base = hint if hint.isidentifier() else "v"
        name = base
        while name in self.names:
            self.counter += 1
            name = f"{base}_{self.counter}"
        self.names.add(name)
        return name

    def lookup(self, name: str, node: ast.AST) -> Any:
        for scope in reversed(self.scopes):
            if name in scope:
                return scope[name]
        if name in self.globals:
            return self.globals[name]
        if hasattr(builtins, name):
            return getattr(builtins, name)
        raise _error(f"name {name!r} is not defined", node)

    def bind(self, name: str, value: Any) -> None:
        if isinstance(value, Mem) and value.origin != "arg" and value.name.startswith("_t"):
            self.names.discard(value.name)
            value.name = self.fresh(name)
        self.scopes[-1][name] = value

    # -- parameters --------------------------------------------------------------------
    def _bind_params(self, runtime_args: Sequence[Any]) -> None:
        fargs = self.fdef.args
        positional = list(fargs.posonlyargs) + list(fargs.args)
        if len(positional) != len(runtime_args):
            raise _error(f"{self.fdef.name} takes {len(positional)} positional arguments, got {len(runtime_args)}")
        mem_dtypes = [_dtype_of(a) for a in runtime_args if _is_memory(a)]
        default_dtype = mem_dtypes[0] if mem_dtypes else "f32"
        for a, value in zip(positional, runtime_args):
            name = a.arg
            self.names.add(name)
            if value is None:
                rank = _annotation_rank(a.annotation)
                if rank is None:
                    raise _error(f"parameter {name!r} is None but is not annotated as Tensor[...]")
                mem = Mem(name, tuple(Sym.dim(name, i) for i in range(rank)), default_dtype, "GM", "arg",
                          optional=True)
                self.params.append(Param(name, "memory", rank, default_dtype, optional=True))
                self.args[name] = mem
                self.scopes[0][name] = mem
            elif _is_memory(value):
                rank = len(tuple(value.shape))
                dtype = _dtype_of(value)
                declared = _annotation_rank(a.annotation)
                if declared is not None and declared != rank:
                    raise _error(f"parameter {name!r}: annotation has rank {declared}, argument has rank {rank}")
                mem = Mem(name, tuple(Sym.dim(name, i) for i in range(rank)), dtype, "GM", "arg",
                          optional=_annotation_rank(a.annotation) is not None and self._may_be_absent(name))
                self.params.append(Param(name, "memory", rank, dtype, optional=mem.optional))
                self.args[name] = mem
                self.scopes[0][name] = mem
            elif isinstance(value, bool):
                raise _error(f"parameter {name!r}: bool arguments are not supported")
            elif isinstance(value, Integral):
                self.params.append(Param(name, "int"))
                self.scopes[0][name] = Sym.arg(name)
            elif isinstance(value, Real):
                self.params.append(Param(name, "float"))
                self.scopes[0][name] = FVal(arg=name)
            else:
                raise _error(f"parameter {name!r}: unsupported runtime argument {type(value).__name__}")

    def _may_be_absent(self, name: str) -> bool:
        """A memory parameter the body tests with `is None` / `is not None` may be absent."""

        for node in ast.walk(self.fdef):
            if isinstance(node, ast.Compare) and len(node.ops) == 1 and isinstance(node.ops[0], (ast.Is, ast.IsNot)):
                if isinstance(node.left, ast.Name) and node.left.id == name:
                    return True
        return False

    # -- statements --------------------------------------------------------------------
    def run(self) -> Func:
        _check_returns(self.fdef.body, self.fdef.name)
        self.exec_block(self.fdef.body)
        return Func(self.fdef.name, self.params, self.args, self.block)

    def exec_block(self, stmts: list[ast.stmt]) -> None:
        for st in stmts:
            if isinstance(st, ast.Return):
                if st.value is not None and not (isinstance(st.value, ast.Constant) and st.value.value is None):
                    raise _error("kernels return nothing", st)
                return
            self.exec_stmt(st)

    def exec_stmt(self, st: ast.stmt) -> None:
        if isinstance(st, ast.Expr):
            if isinstance(st.value, ast.Constant):
                return  # docstring
            self.ev(st.value)
        elif isinstance(st, ast.Assign):
            value = self.ev(st.value)
            for target in st.targets:
                self.assign(target, value, st)
        elif isinstance(st, ast.AnnAssign):
            if st.value is not None:
                self.assign(st.target, self.ev(st.value), st)
        elif isinstance(st, ast.AugAssign):
            if not isinstance(st.target, ast.Name):
                raise _error("augmented assignment needs a name", st)
            current = self.lookup(st.target.id, st)
            self.assign(st.target, self.binop(st.op, current, self.ev(st.value), st), st)
        elif isinstance(st, ast.For):
            self.exec_for(st)
        elif isinstance(st, ast.If):
            self.exec_if(st)
        elif isinstance(st, ast.Pass):
            pass
        else:
            raise _error(f"unsupported statement {type(st).__name__}", st)

    def assign(self, target: ast.expr, value: Any, node: ast.AST) -> None:
        if isinstance(target, ast.Name):
            self.bind(target.id, value)
        elif isinstance(target, (ast.Tuple, ast.List)):
            values = list(value)
            if len(values) != len(target.elts):
                raise _error("unpacking length mismatch", node)
            for t, v in zip(target.elts, values):
                self.assign(t, v, node)
        else:
            raise _error("only names and tuples can be assigned", node)

    def exec_for(self, st: ast.For) -> None:
        call = st.iter
        fn = self.ev(call.func) if isinstance(call, ast.Call) else None
        if getattr(fn, "dsl_op_name", None) != "scf.loop":
            raise _error("for loops iterate over loop(start, end, step)", st)
        if not isinstance(st.target, ast.Name) or st.orelse:
            raise _error("loop target must be one name and the loop has no else", st)
        args = [self.ev(a) for a in call.args]
        if len(args) == 2:
            args.append(1)
        if len(args) != 3 or call.keywords:
            raise _error("loop(start, end, step) takes three positional arguments", st)
        start, end, step = (as_sym(self.to_int(a, st)) for a in args)
        if step.is_const and step.value <= 0:
            raise _error("loop step must be positive", st)
        iv = self.fresh(st.target.id)
        body: list[Op] = []
        op = Op("symbol.for", attrs={"iv": iv, "start": start, "end": end, "step": step}, regions=[body])
        self.block.append(op)
        outer = self.block
        self.block = body
        self.scopes.append({st.target.id: Sym.iv(iv)})
        try:
            self.exec_block(st.body)
        finally:
            self.scopes.pop()
            self.block = outer

    def exec_if(self, st: ast.If) -> None:
        cond = self.ev(st.test)
        if isinstance(cond, (Present, Cmp, _Not)):
            then_b: list[Op] = []
            else_b: list[Op] = []
            self.block.append(Op("scf.if", attrs={"cond": cond}, regions=[then_b, else_b]))
            for branch, stmts in ((then_b, st.body), (else_b, st.orelse)):
                outer = self.block
                self.block = branch
                self.scopes.append({})
                try:
                    self.exec_block(stmts)
                finally:
                    self.scopes.pop()
                    self.block = outer
            return
        if not isinstance(cond, bool):
            raise _error(f"if test must be a Python bool, a presence test or a symbol comparison; got {cond!r}", st)
        self.exec_block(st.body if cond else st.orelse)

    # -- expressions -------------------------------------------------------------------
    def to_int(self, value: Any, node: ast.AST):
        if isinstance(value, Sym):
            return value
        if isinstance(value, bool) or not isinstance(value, Integral):
            raise _error(f"integer expected, got {value!r}", node)
        return int(value)

    def ev(self, node: ast.expr) -> Any:
        if isinstance(node, ast.Constant):
            return node.value
        if isinstance(node, ast.Name):
            return self.lookup(node.id, node)
        if isinstance(node, ast.Attribute):
            base = self.ev(node.value)
            if isinstance(base, Mem):
                if node.attr in ("get_shape", "get_stride"):
                    return _Method(node.attr, base)
                if node.attr == "shape":
                    return list(base.shape)
                raise _error(f"memory has no attribute {node.attr!r}", node)
            return getattr(base, node.attr)
        if isinstance(node, ast.Call):
            return self.call(node)
        if isinstance(node, ast.BinOp):
            return self.binop(node.op, self.ev(node.left), self.ev(node.right), node)
        if isinstance(node, ast.UnaryOp):
            v = self.ev(node.operand)
            if isinstance(node.op, ast.USub):
                return -v
            if isinstance(node.op, ast.UAdd):
                return v
            if isinstance(node.op, ast.Not) and isinstance(v, bool):
                return not v
            raise _error("unsupported unary operation", node)
        if isinstance(node, ast.Compare):
            return self.compare(node)
        if isinstance(node, ast.BoolOp):
            values = [self.ev(v) for v in node.values]
            if not all(isinstance(v, bool) for v in values):
                raise _error("and / or need Python bools", node)
            return all(values) if isinstance(node.op, ast.And) else any(values)
        if isinstance(node, (ast.List, ast.Tuple)):
            return [self.ev(e) for e in node.elts]
        if isinstance(node, ast.Subscript):
            base = self.ev(node.value)
            index = self.ev(node.slice)
            if isinstance(index, Sym):
                if not index.is_const:
                    raise _error("subscripts must be constant", node)
                index = index.value
            return base[index]
        if isinstance(node, ast.IfExp):
            test = self.ev(node.test)
            if not isinstance(test, bool):
                raise _error("conditional expressions need a Python bool test", node)
            return self.ev(node.body if test else node.orelse)
        raise _error(f"unsupported expression {type(node).__name__}", node)

    def binop(self, op: ast.operator, a: Any, b: Any, node: ast.AST) -> Any:
        names = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.FloorDiv: "floordiv", ast.Mod: "mod"}
        if isinstance(a, Sym) or isinstance(b, Sym):
            kind = names.get(type(op))
            if kind is None:
                raise _error("symbolic integers support + - * // %", node)
            return sym_bin(kind, self.to_int(a, node), self.to_int(b, node))
        if isinstance(a, FVal) or isinstance(b, FVal):
            raise _error("float arguments are operands of dma.fill, not of arithmetic", node)
        py = {ast.Add: lambda x, y: x + y, ast.Sub: lambda x, y: x - y, ast.Mult: lambda x, y: x * y,
              ast.FloorDiv: lambda x, y: x // y, ast.Mod: lambda x, y: x % y, ast.Div: lambda x, y: x / y,
              ast.Pow: lambda x, y: x ** y}
        fn = py.get(type(op))
        if fn is None:
            raise _error("unsupported arithmetic", node)
        return fn(a, b)

    def compare(self, node: ast.Compare) -> Any:
        if len(node.ops) != 1:
            raise _error("chained comparisons are not supported", node)
        left = self.ev(node.left)
        right = self.ev(node.comparators[0])
        op = node.ops[0]
        if isinstance(op, (ast.Is, ast.IsNot)):
            if right is not None:
                raise _error("`is` compares with None only", node)
            if isinstance(left, Mem) and left.origin == "arg":
                if not left.optional:
                    # tested inside a called subroutine: the argument may be absent too
                    left.optional = True
                    self.params = [replace(p, optional=True) if p.name == left.name else p for p in self.params]
                return Present(left.name) if isinstance(op, ast.IsNot) else _Not(Present(left.name))
            present = left is not None
            return present if isinstance(op, ast.IsNot) else not present
        kinds = {ast.Eq: "eq", ast.NotEq: "ne", ast.Lt: "lt", ast.LtE: "le", ast.Gt: "gt", ast.GtE: "ge"}
        if isinstance(left, Sym) or isinstance(right, Sym):
            kind = kinds.get(type(op))
            if kind is None:
                raise _error("unsupported symbolic comparison", node)
            return Cmp(kind, as_sym(self.to_int(left, node)), as_sym(self.to_int(right, node)))
        py = {ast.Eq: lambda x, y: x == y, ast.NotEq: lambda x, y: x != y, ast.Lt: lambda x, y: x < y,
              ast.LtE: lambda x, y: x <= y, ast.Gt: lambda x, y: x > y, ast.GtE: lambda x, y: x >= y}
        return py[type(op)](left, right)

    # -- calls -------------------------------------------------------------------------
    def call(self, node: ast.Call) -> Any:
        fn = self.ev(node.func)
        args = [self.ev(a) for a in node.args]
        kwargs = {k.arg: self.ev(k.value) for k in node.keywords}
        if isinstance(fn, _Method):
            if args or kwargs:
                raise _error(f"{fn.name}() takes no arguments", node)
            if fn.name == "get_shape":
                return list(fn.mem.shape)
            raise _error("get_stride is not supported", node)
        if fn is builtins.min or fn is builtins.max:
            values = args[0] if len(args) == 1 else args
            if any(isinstance(v, Sym) for v in values):
                f = smin if fn is builtins.min else smax
                acc = self.to_int(values[0], node)
                for v in values[1:]:
                    acc = f(acc, self.to_int(v, node))
                return acc
            return fn(*values)
        name = getattr(fn, "dsl_op_name", None)
        if name is None:
            if fn in (math.sqrt, float, int, abs, len, range):
                if any(isinstance(a, (Sym, FVal, Mem)) for a in args):
                    raise _error(f"{getattr(fn, '__name__', fn)} of a runtime value is not supported", node)
                return fn(*args, **kwargs)
            if isinstance(fn, types.FunctionType):
                return self.inline(fn, args, kwargs, node)
            raise _error(f"call of {getattr(fn, '__name__', fn)!r} is not a DSL operation", node)
        if name == "scf.loop":
            raise _error("loop() is only valid as a for-loop iterator", node)
        return self.op(name, args, kwargs, node)

    def inline(self, fn: Callable, args: list, kwargs: dict, node: ast.AST) -> Any:
        """A call of a Python function from a kernel body: its body is walked in place,
        with its parameters bound to the caller's values (memories, symbols, float
        operands or plain Python values) and its own globals, so DSL programs can share
        subroutines. The function may return a value with its last statement."""

        if self.depth >= 32:
            raise _error(f"{fn.__name__}: calls nest more than 32 deep", node)
        try:
            source = textwrap.dedent(inspect.getsource(fn))
        except (OSError, TypeError):
            raise _error(f"{fn.__name__}: no source to walk", node) from None
        fdefs = [n for n in ast.parse(source).body if isinstance(n, ast.FunctionDef)]
        if not fdefs:
            raise _error(f"{fn.__name__}: not a function definition", node)
        try:
            bound = inspect.signature(fn).bind(*args, **kwargs)
        except TypeError as exc:
            raise _error(f"{fn.__name__}: {exc}", node) from None
        bound.apply_defaults()
        scope = dict(zip(fn.__code__.co_freevars, (c.cell_contents for c in (fn.__closure__ or ()))))
        scope.update(bound.arguments)
        body = fdefs[0].body
        _check_returns(body, fdefs[0].name)
        saved = self.scopes, self.globals
        self.scopes, self.globals = [scope], fn.__globals__
        self.depth += 1
        try:
            for st in body:
                if isinstance(st, ast.Return):
                    return None if st.value is None else self.ev(st.value)
                self.exec_stmt(st)
            return None
        finally:
            self.depth -= 1
            self.scopes, self.globals = saved

    def mem(self, value: Any, what: str, node: ast.AST) -> Mem:
        if not isinstance(value, Mem):
            raise _error(f"{what} must be a memory value, got {value!r}", node)
        return value

    def syms(self, values: Any, node: ast.AST) -> tuple[Sym, ...]:
        return tuple(as_sym(self.to_int(v, node)) for v in values)

    def new_mem(self, shape, dtype: str, space: str, origin: str = "alloc", source: Mem | None = None) -> Mem:
        return Mem(self.fresh(f"_t{len(self.names)}"), tuple(shape), dtype, space, origin, source)

    def emit(self, name: str, operands: list[Mem], attrs: dict | None = None, result: Mem | None = None) -> Op:
        op = Op(name, operands, attrs or {}, result)
        self.block.append(op)
        return op

    def op(self, name: str, args: list, kwargs: dict, node: ast.AST) -> Any:
        def take(params: Sequence[str], defaults: dict | None = None) -> list:
            values = list(args)
            defaults = defaults or {}
            for p in params[len(values):]:
                if p in kwargs:
                    values.append(kwargs.pop(p))
                elif p in defaults:
                    values.append(defaults[p])
                else:
                    raise _error(f"{name}: missing argument {p!r}", node)
            if kwargs:
                raise _error(f"{name}: unexpected arguments {sorted(kwargs)}", node)
            if len(values) != len(params):
                raise _error(f"{name}: expected {len(params)} arguments, got {len(values)}", node)
            return values

        if name == "dma.alloc":
            shape, dtype, space = take(("shape", "dtype", "space"), {"space": MemorySpace.TSM})
            mem = self.new_mem(self.syms(shape, node), _element(dtype), _space(space))
            self.emit("dma.alloc", [], {}, mem)
            return mem
        if name == "dma.fill":
            target, value = take(("target", "value"))
            self.emit("dma.fill", [self.mem(target, "fill target", node)], {"value": self.fval(value, node)})
            return None
        if name == "dma.view":
            source, offsets, sizes, strides = take(("source", "offsets", "sizes", "strides"))
            src = self.mem(source, "view source", node)
            offsets, sizes, strides = (self.syms(v, node) for v in (offsets, sizes, strides))
            self.check_rank(src, offsets, sizes, strides, name, node)
            mem = self.new_mem(sizes, src.dtype, src.space, "view", src)
            self.emit("dma.view", [src], {"offsets": offsets, "sizes": sizes, "strides": strides}, mem)
            return mem
        if name == "dma.reshape":
            source, shape = take(("source", "shape"))
            src = self.mem(source, "reshape source", node)
            mem = self.new_mem(self.syms(shape, node), src.dtype, src.space, "reshape", src)
            self.emit("dma.reshape", [src], {"shape": mem.shape}, mem)
            return mem
        if name in ("dma.slice", "dma.load"):
            source, offsets, sizes, strides, space = take(("source", "offsets", "sizes", "strides", "space"),
                                                          {"strides": None, "space": None})
            src = self.mem(source, f"{name[4:]} source", node)
            offsets, sizes, strides = self.region(src, offsets, sizes, strides, name, node)
            dst = self.new_mem(sizes, src.dtype, src.space if space is None else _space(space))
            self.emit("dma.alloc", [], {}, dst)
            self.emit(name, [dst, src], {"offsets": offsets, "sizes": sizes, "strides": strides})
            return dst
        if name in ("dma.deslice", "dma.store"):
            target, source, offsets, sizes, strides = take(("target", "source", "offsets", "sizes", "strides"),
                                                           {"strides": None})
            dst = self.mem(target, f"{name[4:]} target", node)
            src = self.mem(source, f"{name[4:]} source", node)
            offsets, sizes, strides = self.region(dst, offsets, sizes, strides, name, node)
            self.emit(name, [dst, src], {"offsets": offsets, "sizes": sizes, "strides": strides})
            return None
        if name == "dma.copy":
            source, space = take(("source", "space"), {"space": None})
            src = self.mem(source, "copy source", node)
            dst = self.new_mem(src.shape, src.dtype, src.space if space is None else _space(space))
            self.emit("dma.alloc", [], {}, dst)
            self.emit("dma.copy", [dst, src])
            return dst
        if name == "dma.cast":
            source, dtype, space = take(("source", "dtype", "memoryspace"), {"memoryspace": None})
            src = self.mem(source, "cast source", node)
            dst = self.new_mem(src.shape, _element(dtype), src.space if space is None else _space(space))
            self.emit("dma.alloc", [], {}, dst)
            self.emit("dma.cast", [dst, src])
            return dst
        if name == "dma.free":
            (value,) = take(("value",))
            mem = self.mem(value, "free operand", node)
            if mem.root().origin == "arg":
                raise _error("dma.free: arguments are owned by the caller; free releases allocated tiles", node)
            self.emit("dma.free", [mem])
            return None
        if name == "dma.flatten":
            (source,) = take(("source",))
            src = self.mem(source, "flatten source", node)
            count = Sym.const(1)
            for d in src.shape:
                count = count * d
            mem = self.new_mem((count,), src.dtype, src.space, "reshape", src)
            self.emit("dma.reshape", [src], {"shape": mem.shape}, mem)
            return mem
        if name == "arch.barrier":
            # each DSL block runs one DSL thread, and every operation ends with a workgroup
            # barrier: the request is kept in the IR and costs one more barrier
            unknown = set(kwargs) - {"visibility", "scope"}
            if args or unknown:
                raise _error("arch.barrier takes the keyword arguments visibility= and scope=", node)
            self.emit("arch.barrier", [])
            return None
        if name in ("arch.get_dynamic_memory", "arch.launch_kernel"):
            raise _error(f"{name} is not supported by the gfx950 front end: tiles are dma.alloc allocations in the "
                         f"workgroup's workspace and a kernel is launched by its entry point", node)
        if name.startswith("arch.get_"):
            take(())
            query = name[len("arch.get_"):]
            if query not in HW_QUERIES:
                raise _error(f"{name} is not a launch query", node)
            return Sym.hw(query)
        if name == "dma.broadcast":
            target, source = take(("target", "source"))
            self.emit("dma.broadcast", [self.mem(target, "broadcast target", node), self.mem(source, "broadcast source", node)])
            return None
        if name == "nn.transpose":
            source, perm = take(("source", "perm"))
            src = self.mem(source, "transpose source", node)
            perm = tuple(int(p) for p in perm)
            if sorted(perm) != list(range(src.rank)):
                raise _error(f"transpose permutation {perm} does not match rank {src.rank}", node)
            dst = self.new_mem(tuple(src.shape[p] for p in perm), src.dtype, src.space)
            self.emit("dma.alloc", [], {}, dst)
            self.emit("dma.transpose", [dst, src], {"perm": perm})
            return dst
        if name == "kernel.matmul":
            out, lhs, rhs, acc = take(("out", "lhs", "rhs", "acc"), {"acc": False})
            mems = [self.mem(v, "matmul operand", node) for v in (out, lhs, rhs)]
            if any(m.rank != 2 for m in mems):
                raise _error("kernel.matmul operands must have rank 2", node)
            if not isinstance(acc, (bool, Cmp)):
                raise _error("matmul acc must be a bool or a symbol comparison", node)
            self.emit("kernel.matmul", mems, {"acc": acc})
            return None
        if name == "kernel.img2col2d":
            out, inp, kh, kw, sh, sw, dh, dw, ph, pw, pl, pr = take(
                ("out", "input", "kh", "kw", "sh", "sw", "dh", "dw", "ph", "pw", "pl", "pr"),
                {"sh": 1, "sw": 1, "dh": 1, "dw": 1, "ph": 0, "pw": 0, "pl": 0, "pr": 0})
            o = self.mem(out, "img2col2d out", node)
            i = self.mem(inp, "img2col2d input", node)
            if i.rank != 4 or o.rank != 6:
                raise _error("img2col2d maps [N,C,H,W] to [N,C,KH,KW,Ho,Wo]", node)
            geo = dict(zip(("kh", "kw", "sh", "sw", "dh", "dw", "ph", "pw", "pl", "pr"),
                           self.syms((kh, kw, sh, sw, dh, dw, ph, pw, pl, pr), node)))
            self.emit("kernel.img2col2d", [o, i], geo)
            return None
        if name == "kernel.exp":
            out, inp = take(("out", "input"))
            self.emit("kernel.exp", [self.mem(out, "exp out", node), self.mem(inp, "exp input", node)])
            return None
        if name == "kernel.reduce":
            out, inp, kind, axis, keepdim = take(("out", "input", "kind", "axis", "keepdim"),
                                                 {"axis": 1, "keepdim": True})
            if not isinstance(kind, KernelReduceKind):
                raise _error("reduce kind must be KernelReduceKind.MAX or SUM", node)
            o, i = self.mem(out, "reduce out", node), self.mem(inp, "reduce input", node)
            if i.rank != 2 or int(axis) != 1 or not keepdim:
                raise _error("kernel.reduce supports rank-2 inputs over axis 1 with keepdim", node)
            self.emit("kernel.reduce", [o, i], {"kind": kind.value, "axis": 1, "keepdim": True})
            return None
        if name == "kernel.binary_elewise" or name in _BINARY_KINDS:
            if name == "kernel.binary_elewise":
                out, lhs, rhs, kind = take(("out", "lhs", "rhs", "kind"))
                if not isinstance(kind, KernelBinaryElewiseKind):
                    raise _error("binary_elewise kind must be a KernelBinaryElewiseKind", node)
                kind = kind.value
            else:
                out, lhs, rhs = take(("out", "lhs", "rhs"))
                kind = _BINARY_KINDS[name]
            mems = [self.mem(v, "elementwise operand", node) for v in (out, lhs, rhs)]
            if len({m.rank for m in mems}) != 1:
                raise _error("elementwise operands must have the same rank", node)
            self.emit("kernel.binary_elewise", mems, {"kind": kind})
            return None
        raise _error(f"DSL operation {name} is not supported by the gfx950 front end", node)

    def fval(self, value: Any, node: ast.AST) -> FVal:
        if isinstance(value, FVal):
            return value
        if isinstance(value, str):
            text = value.strip().lower()
            if text in ("inf", "+inf"):
                return FVal(value=math.inf)
            if text == "-inf":
                return FVal(value=-math.inf)
            raise _error(f"fill value {value!r} is not a number", node)
        if isinstance(value, bool) or not isinstance(value, Real) or isinstance(value, Sym):
            raise _error(f"fill value must be a number or a float argument, got {value!r}", node)
        return FVal(value=float(value))

    def region(self, mem: Mem, offsets, sizes, strides, name: str, node: ast.AST):
        """offsets / sizes / strides of a region of `mem` (strides default to 1)."""

        if strides is None:
            strides = [1] * len(sizes)
        offsets, sizes, strides = (self.syms(v, node) for v in (offsets, sizes, strides))
        self.check_rank(mem, offsets, sizes, strides, name, node)
        return offsets, sizes, strides

    def check_rank(self, mem: Mem, offsets, sizes, strides, name: str, node: ast.AST) -> None:
        if not (len(offsets) == len(sizes) == len(strides) == mem.rank):
            raise _error(f"{name}: offsets/sizes/strides must have rank {mem.rank}", node)


def _check_returns(body: list[ast.stmt], name: str) -> None:
    """A DSL function returns only from its last top-level statement: a return inside a
    loop or a branch would end the walk of that block, not the run-time execution."""

    for i, st in enumerate(body):
        nested = [n for n in ast.walk(st) if isinstance(n, ast.Return)]
        if isinstance(st, ast.Return):
            nested = nested[1:] if i == len(body) - 1 else nested
        if nested:
            raise _error(f"{name}: return is allowed only as the last statement of the function", nested[0])


@dataclass(frozen=True)
class _Not:
    inner: Present

    def __str__(self) -> str:
        return f"!{self.inner}"


def mlir_gen(func_obj: Callable, runtime_args: Sequence[Any]) -> Func:
    """The gfx950 IR of ``func_obj`` specialised to the kinds of ``runtime_args``."""

    return _finish(_Builder.of_function(func_obj, runtime_args).run())


# The reference's DSL modules and the modules of this package that provide the same names.
REFERENCE_MODULES = {
    "kernel_gen.operation": "kernelcode_generate_amd.operation",
    "kernel_gen.operation.arch": "kernelcode_generate_amd.operation.arch",
    "kernel_gen.operation.dma": "kernelcode_generate_amd.operation.dma",
    "kernel_gen.operation.kernel": "kernelcode_generate_amd.operation.kernel",
    "kernel_gen.operation.nn": "kernelcode_generate_amd.operation.nn",
    "kernel_gen.operation.scf": "kernelcode_generate_amd.operation.scf",
    "kernel_gen.symbol_variable.memory": "kernelcode_generate_amd.symbol_variable",
    "kernel_gen.symbol_variable.type": "kernelcode_generate_amd.symbol_variable",
    "kernel_gen.symbol_variable.symbol_dim": "kernelcode_generate_amd.symbol_variable",
}


def source_namespace(source: str, constants: dict | None = None) -> dict:
    """Globals for walking a DSL module given as text, without running it: the names its
    `from kernel_gen... import ...` statements bind, taken from this package's modules of
    the same role (REFERENCE_MODULES), plus ``constants`` for the module-level values its
    kernels read (tile sizes, pads, seeds' draws). Other imports are left out: a kernel
    body that used them fails with a name error."""

    import importlib

    namespace: dict = dict(constants or {})
    for node in ast.parse(source).body:
        if isinstance(node, ast.ImportFrom) and node.module in REFERENCE_MODULES:
            module = importlib.import_module(REFERENCE_MODULES[node.module])
            for alias in node.names:
                if hasattr(module, alias.name):
                    namespace[alias.asname or alias.name] = getattr(module, alias.name)
                elif alias.name in ("kernel", "dma", "nn", "scf", "arch"):
                    namespace[alias.asname or alias.name] = importlib.import_module(f"{module.__name__}.{alias.name}")
    return namespace


def mlir_gen_source(source: str, function: str, runtime_args: Sequence[Any], constants: dict | None = None) -> Func:
    """The gfx950 IR of the DSL function ``function`` defined in the module text
    ``source`` (walked, never executed), specialised to the kinds of ``runtime_args``;
    names resolve through ``source_namespace(source, constants)``."""

    fdefs = [n for n in ast.parse(source).body if isinstance(n, ast.FunctionDef) and n.name == function]
    if not fdefs:
        raise _error(f"no function {function!r} in the source")
    return _finish(_Builder(fdefs[0], source_namespace(source, constants), {}, runtime_args).run())


def _finish(func: Func) -> Func:
    for op in func.walk():
        if op.name == "scf.if" and isinstance(op.attrs["cond"], _Not):
            op.attrs["cond"] = op.attrs["cond"].inner
            op.regions.reverse()
    return func


__all__ = ["REFERENCE_MODULES", "mlir_gen", "mlir_gen_source", "source_namespace"]
