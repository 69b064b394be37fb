"""Tracing IR behind the ``T.*`` surface.

The reference parses ``@T.prim_func`` bodies with TVMScript into TIR (tilelang/language/parser,
src/ir.cc). This build has no TIR: a prim_func body is *executed once* with symbolic stand-ins
(grid/loop variables, buffers) and every tile op it issues is recorded. The recorded trace is
matched against the operator families that have gfx950 kernels (tilelang/jit/adapter/mi355x/
recognize.py); there is no general code generation.

Semantics kept from the reference:
  * ``T.Kernel(*extents)`` yields one variable per grid dim (src/ir.cc:155-220); with
    ``is_cpu=True`` the reference runs the grid serially (ir.cc:164-173) — for the trace both
    are the same: the body is recorded once with symbolic block indices.
  * ``T.Pipelined/serial/Parallel`` loops run their body once with a symbolic induction var;
    the extent expression is kept (causal FA is recognised from it).
  * Python ``if`` on a symbolic condition (e.g. ``if kr == 0:`` in
    examples/deepseek_mla/example_mla_decode_paged.py:77) records the condition and traces the
    then-branch.
  * Buffer regions follow RegionOp (src/op/op.cc:54-69): a point index is the region's base,
    the extents come from the other operand of the copy.
"""
from __future__ import annotations

import math
import threading
from typing import Any, List, Optional, Sequence, Tuple

_tls = threading.local()


def current_tracer() -> Optional["Tracer"]:
    return getattr(_tls, "tracer", None)


# ------------------------------------------------------------------------------------------------
# dtypes

_DTYPE_ALIASES = {
    "float": "float32",
    "float32": "float32",
    "fp32": "float32",
    "float16": "float16",
    "half": "float16",
    "fp16": "float16",
    "bfloat16": "bfloat16",
    "bf16": "bfloat16",
    "float64": "float64",
    "int32": "int32",
    "int64": "int64",
    "int8": "int8",
    "uint8": "uint8",
    "uint32": "uint32",
    "bool": "bool",
    "float8_e4m3": "float8_e4m3",
    "float8_e4m3fn": "float8_e4m3",
    "e4m3_float8": "float8_e4m3",
    "float8_e5m2": "float8_e5m2",
    "e5m2_float8": "float8_e5m2",
}


def canon_dtype(dtype: Any) -> str:
    """Normalise a dtype spelling ("float", "e4m3_float8", torch.float16, ...) to one name."""
    if hasattr(dtype, "is_floating_point") or str(type(dtype)) == "<class 'torch.dtype'>":
        name = str(dtype).replace("torch.", "")
    else:
        name = str(dtype)
    if name not in _DTYPE_ALIASES:
        raise ValueError(f"unsupported dtype {dtype!r}")
    return _DTYPE_ALIASES[name]


# ------------------------------------------------------------------------------------------------
# Expressions


class Expr:
    """A symbolic scalar expression recorded during tracing."""

    __slots__ = ("op", "args", "dtype")

    def __init__(self, op: str, args: Sequence[Any] = (), dtype: Optional[str] = None):
        self.op = op
        self.args = tuple(args)
        self.dtype = dtype

    # arithmetic -----------------------------------------------------------------------------
    def _bin(self, op, other, rev=False):
        a, b = (other, self) if rev else (self, other)
        return binop(op, a, b)

    def __add__(self, o):
        return self._bin("add", o)

    def __radd__(self, o):
        return self._bin("add", o, True)

    def __sub__(self, o):
        return self._bin("sub", o)

    def __rsub__(self, o):
        return self._bin("sub", o, True)

    def __mul__(self, o):
        return self._bin("mul", o)

    def __rmul__(self, o):
        return self._bin("mul", o, True)

    def __truediv__(self, o):
        return self._bin("div", o)

    def __rtruediv__(self, o):
        return self._bin("div", o, True)

    def __floordiv__(self, o):
        return self._bin("floordiv", o)

    def __rfloordiv__(self, o):
        return self._bin("floordiv", o, True)

    def __mod__(self, o):
        return self._bin("mod", o)

    def __rmod__(self, o):
        return self._bin("mod", o, True)

    def __neg__(self):
        if self.op == "const":
            return Const(-self.args[0], self.dtype)
        return Expr("neg", (self,), self.dtype)

    def __pos__(self):
        return self

    # comparisons ----------------------------------------------------------------------------
    def __lt__(self, o):
        return self._bin("lt", o)

    def __le__(self, o):
        return self._bin("le", o)

    def __gt__(self, o):
        return self._bin("gt", o)

    def __ge__(self, o):
        return self._bin("ge", o)

    def __eq__(self, o):  # noqa: D401 - symbolic equality
        return self._bin("eq", o)

    def __ne__(self, o):
        return self._bin("ne", o)

    def __and__(self, o):
        return self._bin("and", o)

    def __or__(self, o):
        return self._bin("or", o)

    __hash__ = object.__hash__

    def __bool__(self):
        if self.op == "const":
            return bool(self.args[0])
        tr = current_tracer()
        if tr is not None:
            tr.record("branch", (self,), {})
        # The then-branch is the one traced.
        return True

    def __index__(self):
        if self.op == "const" and isinstance(self.args[0], int):
            return self.args[0]
        raise TypeError(f"symbolic expression {self!r} has no static integer value")

    def __int__(self):
        return self.__index__()

    def __float__(self):
        if self.op == "const":
            return float(self.args[0])
        raise TypeError(f"symbolic expression {self!r} has no static value")

    # inspection -----------------------------------------------------------------------------
    def walk(self):
        yield self
        for a in self.args:
            if isinstance(a, Expr):
                yield from a.walk()

    def free_vars(self) -> set:
        return {e.args[0] for e in self.walk() if e.op == "var"}

    def consts(self) -> List[float]:
        return [e.args[0] for e in self.walk() if e.op == "const"]

    def has_op(self, op: str) -> bool:
        return any(e.op == op for e in self.walk())

    def __repr__(self):
        if self.op == "var":
            return str(self.args[0])
        if self.op == "const":
            return repr(self.args[0])
        if self.op == "load":
            return f"{self.args[0].name}[{', '.join(map(repr, self.args[1]))}]"
        return f"{self.op}({', '.join(map(repr, self.args))})"


class Var(Expr):
    """Grid or loop variable. Iterable so that ``as (bx,)`` unpacks a 1-D grid."""

    __slots__ = ()

    def __init__(self, name: str, dtype: str = "int32"):
        super().__init__("var", (name,), dtype)

    @property
    def name(self) -> str:
        return self.args[0]

    def __iter__(self):
        return iter((self,))


class SymVar(Var):
    """Symbolic shape variable (``T.symbolic``, reference tilelang/language/__init__.py:85-86):
    a tensor extent bound when the kernel is called (from the argument's shape); the traced
    program is specialised to the bound values before recognition."""

    __slots__ = ()


class ScalarParam(Var):
    """Scalar prim_func parameter (``max_seqlen_q: T.int32``): a symbolic value in the traced
    body and a Python number at call time (the reference passes such parameters as plain
    integers, tilelang/jit/adapter/cython/cython_wrapper.pyx:117-122)."""

    __slots__ = ()
    scope = "scalar"
    shape = ()
    ndim = 0


def Const(value, dtype: Optional[str] = None) -> Expr:
    return Expr("const", (value,), dtype)


def is_const(x) -> bool:
    return isinstance(x, (int, float)) or (isinstance(x, Expr) and x.op == "const")


def const_value(x):
    if isinstance(x, Expr):
        if x.op != "const":
            raise TypeError(f"{x!r} is not constant")
        return x.args[0]
    return x


_FOLD = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "div": lambda a, b: a / b,
    "floordiv": lambda a, b: a // b,
    "mod": lambda a, b: a % b,
    "lt": lambda a, b: a < b,
    "le": lambda a, b: a <= b,
    "gt": lambda a, b: a > b,
    "ge": lambda a, b: a >= b,
    "eq": lambda a, b: a == b,
    "ne": lambda a, b: a != b,
    "and": lambda a, b: a and b,
    "or": lambda a, b: a or b,
    "min": min,
    "max": max,
}


_FOLD_CALL = dict(_FOLD, ceildiv=lambda a, b: -(-a // b))


def sym_names(x) -> set:
    """Names of the symbolic shape variables in an expression (or a plain value)."""
    if isinstance(x, Expr):
        return {e.args[0] for e in x.walk() if isinstance(e, SymVar)}
    return set()


def substitute(x, env: dict, memo: Optional[dict] = None):
    """``x`` with the symbolic shape variables named in ``env`` replaced by their values and
    the arithmetic over them folded. Buffers, accesses, loops and launches that mention one are
    rebuilt (one new object per old one, so identities between trace records are kept); every
    other object is returned as is."""
    memo = {} if memo is None else memo
    key = id(x)
    if key in memo:
        return memo[key]
    out = x
    if isinstance(x, SymVar):
        if x.args[0] in env:
            out = Const(int(env[x.args[0]]), x.dtype)
    elif isinstance(x, BufferAccess):
        b = substitute(x.buffer, env, memo)
        idx = substitute(x.indices, env, memo)
        if b is not x.buffer or idx is not x.indices:
            out = BufferAccess(b, idx)
    elif isinstance(x, Expr):
        if sym_names(x) & set(env):
            args = tuple(substitute(a, env, memo) for a in x.args)
            if all(is_const(a) for a in args) and x.op in _FOLD_CALL and len(args) == 2:
                out = binop(x.op, args[0], args[1]) if x.op in _FOLD else \
                    Const(_FOLD_CALL[x.op](*(const_value(a) for a in args)), x.dtype)
            else:
                out = Expr(x.op, args, x.dtype)
    elif isinstance(x, Buffer):
        shape = substitute(tuple(x.shape), env, memo)
        if shape is not x.shape and any(a is not b for a, b in zip(shape, x.shape)):
            out = Buffer.__new__(Buffer)
            out.__dict__.update(x.__dict__)
            out.shape = tuple(shape)
    elif isinstance(x, tuple):
        items = tuple(substitute(a, env, memo) for a in x)
        out = x if all(a is b for a, b in zip(items, x)) else items
    elif isinstance(x, list):
        items = [substitute(a, env, memo) for a in x]
        out = x if all(a is b for a, b in zip(items, x)) else items
    elif isinstance(x, dict):
        items = {k: substitute(v, env, memo) for k, v in x.items()}
        out = x if all(items[k] is x[k] for k in x) else items
    elif isinstance(x, slice):
        st, sp, se = (substitute(v, env, memo) for v in (x.start, x.stop, x.step))
        if st is not x.start or sp is not x.stop or se is not x.step:
            out = slice(st, sp, se)
    elif isinstance(x, Loop):
        ext = substitute(x.extents, env, memo)
        kw = substitute(x.kwargs, env, memo)
        if ext is not x.extents or kw is not x.kwargs:
            out = Loop(x.kind, x.vars, ext, kw)
    elif isinstance(x, KernelLaunch):
        ext = substitute(x.extents, env, memo)
        if ext is not x.extents:
            out = KernelLaunch(x.index, ext, x.threads, x.is_cpu, x.vars)
    elif isinstance(x, Op):
        args = substitute(x.args, env, memo)
        kw = substitute(x.kwargs, env, memo)
        loops = substitute(x.loops, env, memo)
        if args is not x.args or kw is not x.kwargs or loops is not x.loops:
            out = Op(x.name, args, kw, loops, x.kernel)
    memo[key] = out
    return out


def binop(op: str, a, b):
    """Build ``op(a, b)``, folding when both sides are constants."""
    if is_const(a) and is_const(b):
        va, vb = const_value(a), const_value(b)
        try:
            v = _FOLD[op](va, vb)
        except ZeroDivisionError:
            v = math.inf
        dt = a.dtype if isinstance(a, Expr) else (b.dtype if isinstance(b, Expr) else None)
        return Const(v, dt)
    dt = a.dtype if isinstance(a, Expr) else (b.dtype if isinstance(b, Expr) else None)
    return Expr(op, (wrap(a), wrap(b)), dt)


def wrap(x):
    if isinstance(x, Expr):
        return x
    if isinstance(x, (bool, int, float)):
        return Const(x)
    return x


def call(op: str, *args, dtype: Optional[str] = None) -> Expr:
    return Expr(op, tuple(wrap(a) for a in args), dtype)


# ------------------------------------------------------------------------------------------------
# Buffers


class TensorType:
    """Annotation object of ``T.Tensor(shape, dtype)`` (a parameter's static type)."""

    def __init__(self, shape, dtype="float32"):
        if isinstance(shape, int):
            shape = (shape,)
        self.shape = tuple(shape)
        self.dtype = canon_dtype(dtype)

    def __repr__(self):
        return f"Tensor({list(self.shape)}, {self.dtype})"


class Buffer:
    """A named tensor: a prim_func parameter (scope "global") or a tile allocation."""

    _counter = 0

    def __init__(self, name: str, shape, dtype: str, scope: str):
        if isinstance(shape, int):
            shape = (shape,)
        self.name = name
        self.shape = tuple(shape)
        self.dtype = canon_dtype(dtype)
        self.scope = scope

    @property
    def ndim(self):
        return len(self.shape)

    def __getitem__(self, idx) -> "BufferAccess":
        if not isinstance(idx, tuple):
            idx = (idx,)
        return BufferAccess(self, idx)

    def __setitem__(self, idx, value):
        if not isinstance(idx, tuple):
            idx = (idx,)
        tr = current_tracer()
        if tr is not None:
            tr.record("store", (self, idx, wrap(value)), {})

    def numel(self):
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    def __repr__(self):
        return f"{self.name}<{self.scope} {list(self.shape)} {self.dtype}>"

    __hash__ = object.__hash__

    def __eq__(self, other):
        return self is other


class BufferAccess(Expr):
    """``buf[idx]``: a scalar load in expressions and a region in tile copies."""

    __slots__ = ()

    def __init__(self, buffer: Buffer, indices: Tuple[Any, ...]):
        super().__init__("load", (buffer, tuple(indices)), buffer.dtype)

    @property
    def buffer(self) -> Buffer:
        return self.args[0]

    @property
    def indices(self):
        return self.args[1]

    def region(self, fallback_extents: Optional[Sequence[int]] = None):
        """Return (starts, extents). Point indices take extents from ``fallback_extents``
        aligned to the trailing dims (RegionOp, src/op/op.cc:54-69)."""
        starts, extents = [], []
        for d, ix in enumerate(self.indices):
            if isinstance(ix, slice):
                st = 0 if ix.start is None else ix.start
                sp = self.buffer.shape[d] if ix.stop is None else ix.stop
                starts.append(st)
                extents.append(binop("sub", sp, st))
            else:
                starts.append(ix)
                extents.append(None)
        # An access with a slice is a region whose point indices span one element; an access of
        # point indices only takes the tile's extents on its trailing dims and 1 on the leading
        # ones (tilelang/language/copy.py:40-62).
        if fallback_extents is not None and all(e is None for e in extents):
            fb = list(fallback_extents)
            j = len(fb) - 1
            for d in range(len(extents) - 1, -1, -1):
                extents[d] = fb[j] if j >= 0 else 1
                j -= 1
        extents = [1 if e is None else e for e in extents]
        return starts, extents


def as_region(x):
    """Normalise a copy operand to (buffer, starts, extents or None)."""
    if isinstance(x, Buffer):
        return x, [0] * x.ndim, list(x.shape)
    if isinstance(x, BufferAccess):
        st, ex = x.region()
        return x.buffer, st, ex
    raise TypeError(f"expected a buffer or buffer region, got {x!r}")


# ------------------------------------------------------------------------------------------------
# Trace records


class Op:
    """One recorded statement: ``name(*args, **kwargs)`` inside ``loops`` of kernel ``kernel``."""

    __slots__ = ("name", "args", "kwargs", "loops", "kernel")

    def __init__(self, name, args, kwargs, loops, kernel):
        self.name = name
        self.args = args
        self.kwargs = kwargs
        self.loops = loops
        self.kernel = kernel

    def __repr__(self):
        return f"Op({self.name}, k={self.kernel}, loops={[l.kind for l in self.loops]})"


class Loop:
    __slots__ = ("kind", "vars", "extents", "kwargs")

    def __init__(self, kind, vars_, extents, kwargs):
        self.kind = kind
        self.vars = vars_
        self.extents = extents
        self.kwargs = kwargs


class KernelLaunch:
    __slots__ = ("index", "extents", "threads", "is_cpu", "vars")

    def __init__(self, index, extents, threads, is_cpu, vars_):
        self.index = index
        self.extents = extents
        self.threads = threads
        self.is_cpu = is_cpu
        self.vars = vars_


class Tracer:
    def __init__(self):
        self.ops: List[Op] = []
        self.kernels: List[KernelLaunch] = []
        self.allocs: List[Buffer] = []
        self._loops: List[Loop] = []
        self._kernel: Optional[KernelLaunch] = None
        self._prev = None

    def __enter__(self):
        self._prev = current_tracer()
        _tls.tracer = self
        return self

    def __exit__(self, *exc):
        _tls.tracer = self._prev
        return False

    def record(self, name, args, kwargs):
        k = self._kernel.index if self._kernel is not None else -1
        self.ops.append(Op(name, tuple(args), dict(kwargs), tuple(self._loops), k))

    def push_loop(self, loop: Loop):
        self._loops.append(loop)
        self.record("loop_begin", (loop,), {})

    def pop_loop(self):
        loop = self._loops.pop()
        self.record("loop_end", (loop,), {})

    def begin_kernel(self, extents, threads, is_cpu):
        names = ("bx", "by", "bz")
        vars_ = tuple(Var(names[i] if i < 3 else f"b{i}") for i in range(len(extents)))
        kl = KernelLaunch(len(self.kernels), tuple(extents), threads, is_cpu, vars_)
        self.kernels.append(kl)
        self._kernel = kl
        return kl

    def end_kernel(self):
        self._kernel = None

    def alloc(self, buf: Buffer):
        self.allocs.append(buf)
        self.record("alloc", (buf,), {})
        return buf


def record(name: str, *args, **kwargs):
    tr = current_tracer()
    if tr is None:
        raise RuntimeError(f"T.{name} used outside of a @T.prim_func body")
    tr.record(name, args, kwargs)


def fresh_name(prefix: str) -> str:
    Buffer._counter += 1
    return f"{prefix}_{Buffer._counter}"
