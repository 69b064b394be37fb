"""``tilelang.language`` (imported as ``T``): the kernel-description surface.

Names follow the reference: the BM1690 tile intrinsics ``T.ppl_*``
(reference tilelang/language/customize.py:101-603), the upstream tile ops the MLA example uses
(``T.copy/gemm/fill/clear/reduce_*``), grid/loop frames (tilelang/language/kernel.py:186-235,
pipeline.py), allocation (allocate.py) and scalar math. Every call is recorded by the tracer in
``ir.py``; nothing is lowered or code-generated here.
"""
from __future__ import annotations

import builtins as _builtins
import enum
import functools
import inspect
import math
from typing import Any, Optional

from . import ir
from .ir import (Buffer, BufferAccess, Const, Expr, Loop, TensorType, Tracer, Var, binop, call,
                 canon_dtype, current_tracer, record, wrap)

# ------------------------------------------------------------------------------------------------
# Types


def Tensor(shape, dtype="float32", *args, **kwargs) -> TensorType:
    """Parameter annotation ``T.Tensor(shape, dtype)``."""
    return TensorType(shape, dtype)


Buffer_ = Tensor
Buffer = Tensor  # noqa: F811  (T.Buffer is an alias of T.Tensor in annotations)
# macro argument annotations (tile buffers passed to a @T.macro); inlining ignores them
SharedBuffer = Tensor
FragmentBuffer = Tensor
LocalBuffer = Tensor


class PrimFunc:
    """A traced kernel program: its parameters and the recorded op trace."""

    def __init__(self, name, params, tracer: Tracer, fn):
        self.name = name
        self.params = params
        self.ops = tracer.ops
        self.kernels = tracer.kernels
        self.allocs = tracer.allocs
        self.fn = fn
        self.attrs = {"global_symbol": name}

    def __repr__(self):
        ps = ", ".join(repr(p) for p in self.params)
        return f"PrimFunc {self.name}({ps}) [{len(self.ops)} ops, {len(self.kernels)} kernels]"

    def symbolic_vars(self) -> list:
        """Names of the symbolic shape variables of the parameters (T.symbolic), in order of
        first appearance."""
        names = []
        for p in self.params:
            for d in getattr(p, "shape", ()):
                for n in sorted(ir.sym_names(d)):
                    if n not in names:
                        names.append(n)
        return names

    def specialize(self, env: dict) -> "PrimFunc":
        """This program with its symbolic shape variables bound to the integers in ``env`` (the
        trace is re-written with the values folded in; nothing is re-executed)."""
        memo: dict = {}
        out = PrimFunc.__new__(PrimFunc)
        out.name = self.name
        out.params = [ir.substitute(p, env, memo) for p in self.params]
        out.ops = [ir.substitute(o, env, memo) for o in self.ops]
        out.kernels = [ir.substitute(k, env, memo) for k in self.kernels]
        out.allocs = [ir.substitute(b, env, memo) for b in self.allocs]
        out.fn = self.fn
        out.attrs = dict(self.attrs)
        return out

    def script(self) -> str:
        lines = [repr(self)]
        for op in self.ops:
            if op.name in ("loop_begin", "loop_end", "alloc"):
                continue
            lines.append(f"  k{op.kernel} {'  ' * len(op.loops)}{op.name}")
        return "\n".join(lines)


def prim_func(fn=None, *, private: bool = False, check_well_formed: bool = False):
    """Trace ``fn`` into a :class:`PrimFunc`.

    Parameters are annotated ``T.Tensor(shape, dtype)`` or a scalar type such as ``T.int32``;
    the annotations are evaluated when the function is defined (as TVMScript does), then the body
    runs once with symbolic buffers and scalars.
    """

    def deco(f):
        sig = inspect.signature(f)
        params = []
        for name, p in sig.parameters.items():
            ann = p.annotation
            scalar_dt = getattr(ann, "_scalar_dtype", None)
            if scalar_dt is not None:
                params.append(ir.ScalarParam(name, scalar_dt))
                continue
            if not isinstance(ann, TensorType):
                raise TypeError(
                    f"prim_func {f.__name__}: parameter {name!r} must be annotated "
                    f"T.Tensor(shape, dtype) or a scalar type such as T.int32")
            params.append(ir.Buffer(name, ann.shape, ann.dtype, "global"))
        tracer = Tracer()
        with tracer:
            f(*params)
        return PrimFunc(f.__name__, params, tracer, f)

    if fn is None:
        return deco
    return deco(fn)


def symbolic(name: str, dtype: str = "int32"):
    """A symbolic tensor extent (reference tilelang/language/__init__.py:85-86): usable in
    ``T.Tensor`` shapes and in the body's arithmetic; bound from the arguments' shapes when the
    compiled kernel is called."""
    return ir.SymVar(name, canon_dtype(dtype))


def macro(fn=None, **kwargs):
    """``@T.macro``: inlined at trace time (the body simply runs at each call)."""

    def deco(f):
        @functools.wraps(f)
        def inner(*a, **k):
            return f(*a, **k)

        return inner

    if fn is None:
        return deco
    return deco(fn)


# ------------------------------------------------------------------------------------------------
# Frames


class _KernelFrame:

    def __init__(self, extents, threads, is_cpu, prelude):
        self.extents = tuple(wrap(e) if isinstance(e, Expr) else e for e in extents)
        self.threads = threads
        self.is_cpu = is_cpu
        self.launch = None

    def __enter__(self):
        tr = current_tracer()
        if tr is None:
            raise RuntimeError("T.Kernel used outside of a @T.prim_func body")
        self.launch = tr.begin_kernel(self.extents, self.threads, self.is_cpu)
        v = self.launch.vars
        return v[0] if len(v) == 1 else v

    def __exit__(self, *exc):
        current_tracer().end_kernel()
        return False


def Kernel(*extents, threads=None, is_cpu: bool = False, prelude=None, **kwargs):
    """Grid frame (reference tilelang/language/kernel.py:186-235)."""
    if len(extents) == 1 and isinstance(extents[0], (list, tuple)):
        extents = tuple(extents[0])
    return _KernelFrame(extents, threads, is_cpu, prelude)


def _loop(kind, extents, names, **kwargs):
    tr = current_tracer()
    if tr is None:
        raise RuntimeError(f"T.{kind} used outside of a @T.prim_func body")
    vars_ = tuple(Var(n) for n in names)
    tr.push_loop(Loop(kind, vars_, tuple(extents), kwargs))
    try:
        yield vars_[0] if len(vars_) == 1 else vars_
    finally:
        tr.pop_loop()


_loop_id = [0]


def _names(prefix, n):
    _loop_id[0] += 1
    return [f"{prefix}{_loop_id[0]}_{i}" for i in range(n)]


def Pipelined(start, stop=None, num_stages: int = 0, order=None, stage=None, sync=None,
              group=None):
    extent = start if stop is None else binop("sub", stop, start)
    return _loop("pipelined", (extent,), _names("k", 1), num_stages=num_stages)


def serial(start, stop=None, step=None):
    extent = start if stop is None else binop("sub", stop, start)
    return _loop("serial", (extent,), _names("s", 1))


def unroll(start, stop=None, step=None):
    return serial(start, stop, step)


def Parallel(*extents, coalesced_width=None):
    return _loop("parallel", extents, _names("p", len(extents)))


def grid(*extents):
    return _loop("grid", extents, _names("g", len(extents)))


# ------------------------------------------------------------------------------------------------
# Allocation (reference tilelang/language/allocate.py)


def _alloc(shape, dtype, scope):
    tr = current_tracer()
    buf = ir.Buffer(ir.fresh_name(scope), shape, dtype, scope)
    if tr is not None:
        tr.alloc(buf)
    return buf


def alloc_shared(shape, dtype, scope="shared.dyn"):
    return _alloc(shape, dtype, "shared")


def alloc_fragment(shape, dtype, scope="local.fragment"):
    return _alloc(shape, dtype, "fragment")


def alloc_local(shape, dtype, scope="local"):
    return _alloc(shape, dtype, "local")


# ------------------------------------------------------------------------------------------------
# BM1690 tile intrinsics (reference tilelang/language/customize.py:101-603; semantics of each
# in src/target/codegen_ppl.cc, cited per op).


def ppl_gemm(A, B, C, transpose_A=False, transpose_B=False):
    """C += A @ B (fp32 C) or C = A @ B^T (codegen_ppl.cc:1244-1279)."""
    record("ppl_gemm", A, B, C, transpose_A=transpose_A, transpose_B=transpose_B)


def ppl_copy(src, dst, *args, **kwargs):
    """Tile copy with optional cast, round-half-even (codegen_ppl.cc:961-1198)."""
    record("ppl_copy", src, dst)


def ppl_fill(buffer, value):
    record("ppl_fill", buffer, wrap(value))


def ppl_clear(buffer):
    record("ppl_fill", buffer, Const(0.0))


def ppl_add(out, inp1, inp2):
    record("ppl_add", out, inp1, inp2)


def ppl_subtract(out, inp1, inp2):
    record("ppl_sub", out, inp1, inp2)


ppl_sub = ppl_subtract


def ppl_mul(out, inp1, inp2):
    record("ppl_mul", out, inp1, inp2)


def ppl_div(out, inp1, inp2):
    record("ppl_div", out, inp1, inp2)


def ppl_add_C(out, inp1, value):
    record("ppl_add_C", out, inp1, wrap(value))


def ppl_mul_C(out, inp1, value):
    record("ppl_mul_C", out, inp1, wrap(value))


def ppl_exp2(out, work0=None, work1=None, coeff=None, table=None):
    """Natural exponential in place, fp32 (customize.py:313-339 docstring; codegen :1294-1320)."""
    record("ppl_exp", out)


def ppl_rsqrt(out, inp):
    record("ppl_rsqrt", out, inp)


def ppl_reduce_sum(inp, out, dim=1):
    record("ppl_reduce_sum", inp, out, dim=dim)


def ppl_reduce_max(inp, out, dim=1, clear=True):
    record("ppl_reduce_max", inp, out, dim=dim, clear=clear)


def ppl_rope_add(out, even_inp1, even_inp2, odd_inp1, odd_inp2):
    """out[2i] = e1[2i] + e2[2i+1]; out[2i+1] = o1[2i+1] + o2[2i] (codegen_ppl.cc:1809-1848)."""
    record("ppl_rope_add", out, even_inp1, even_inp2, odd_inp1, odd_inp2)


def ppl_sigmoid(out, inp, work0=None, work1=None, coeff=None, table=None):
    record("ppl_sigmoid", out, inp)


def ppl_gather(output, param, index, param_h):
    record("ppl_gather", output, param, index, param_h)


def ppl_topk(dst_data, dst_idx, src, K, descended, length):
    record("ppl_topk", dst_data, dst_idx, src, K, descended, length)


# ------------------------------------------------------------------------------------------------
# Upstream tile ops (used by examples/deepseek_mla and examples/flash_attention)


class GemmWarpPolicy(enum.IntEnum):
    Square = 0
    FullRow = 1
    FullCol = 2


def copy(src, dst, *args, **kwargs):
    record("copy", src, dst)


def gemm(A, B, C, transpose_A=False, transpose_B=False, policy=GemmWarpPolicy.Square, k_pack=1,
         wg_wait=0, **kwargs):
    """C += A @ op(B) with fp32 accumulation (upstream semantics: accumulate)."""
    record("gemm", A, B, C, transpose_A=transpose_A, transpose_B=transpose_B)


def fill(buffer, value):
    record("fill", buffer, wrap(value))


def clear(buffer):
    record("fill", buffer, Const(0.0))


def reduce_max(buffer, out, dim=-1, clear=True):
    record("reduce_max", buffer, out, dim=dim, clear=clear)


def reduce_sum(buffer, out, dim=-1, clear=True):
    record("reduce_sum", buffer, out, dim=dim, clear=clear)


def reduce_min(buffer, out, dim=-1, clear=True):
    record("reduce_min", buffer, out, dim=dim, clear=clear)


def reduce_abssum(buffer, out, dim=-1):
    record("reduce_abssum", buffer, out, dim=dim)


def use_swizzle(panel_size: int = 8, order: str = "row", enable: bool = True):
    """Block-rasterisation hint; kernels here choose their own tile order."""
    return None


def annotate_layout(layout_map):
    """Layout annotations are accepted; the gfx950 kernels use fixed LDS layouts."""
    return None


def annotate_padding(padding_map):
    return None


class Fragment:
    """Stand-in for tilelang.layout.Fragment in ``T.annotate_layout`` maps."""

    def __init__(self, shape=None, forward_thread_fn=None, replicate=1, forward_fn=None,
                 forward_index_fn=None, **kwargs):
        self.shape = shape


class Layout(Fragment):
    pass


def no_set_max_nreg():
    return None


def disable_warp_group_reg_alloc():
    return None


# ------------------------------------------------------------------------------------------------
# Scalar math


def _dt_ctor(dtype):

    def ctor(value=0, *args, **kwargs):
        if isinstance(value, Expr):
            return Expr("cast", (value,), dtype)
        if dtype.startswith("int"):
            return Const(int(value), dtype)
        return Const(float(value), dtype)

    ctor.__name__ = dtype
    ctor._scalar_dtype = dtype  # usable as a scalar parameter annotation
    return ctor


float16 = _dt_ctor("float16")
float32 = _dt_ctor("float32")
float64 = _dt_ctor("float64")
bfloat16 = _dt_ctor("bfloat16")
int32 = _dt_ctor("int32")
int64 = _dt_ctor("int64")
int8 = _dt_ctor("int8")
uint8 = _dt_ctor("uint8")
boolean = _dt_ctor("bool")


def cast(value, dtype):
    return Expr("cast", (wrap(value),), canon_dtype(dtype))


def infinity(dtype="float32"):
    return Const(math.inf, canon_dtype(dtype))


def max_value(dtype="float32"):
    return Const(3.4028234663852886e38, canon_dtype(dtype))


def min_value(dtype="float32"):
    return Const(-3.4028234663852886e38, canon_dtype(dtype))


def ceildiv(a, b):
    if ir.is_const(a) and ir.is_const(b):
        va, vb = ir.const_value(a), ir.const_value(b)
        return (va + vb - 1) // vb
    return call("ceildiv", a, b)


def floordiv(a, b):
    return binop("floordiv", a, b)


def floormod(a, b):
    return binop("mod", a, b)


def truncdiv(a, b):
    return binop("floordiv", a, b)


def truncmod(a, b):
    return binop("mod", a, b)


def min(a, b):  # noqa: A001 - TIR name
    if ir.is_const(a) and ir.is_const(b):
        return Const(_builtins.min(ir.const_value(a), ir.const_value(b)))
    return call("min", a, b)


def max(a, b):  # noqa: A001 - TIR name
    if ir.is_const(a) and ir.is_const(b):
        return Const(_builtins.max(ir.const_value(a), ir.const_value(b)))
    return call("max", a, b)


def if_then_else(cond, then_value, else_value):
    return call("if_then_else", cond, then_value, else_value)


def Select(cond, then_value, else_value):
    return if_then_else(cond, then_value, else_value)


def exp2(x):
    return call("exp2", x)


def exp(x):
    return call("exp", x)


def log2(x):
    return call("log2", x)


def log(x):
    return call("log", x)


def sqrt(x):
    return call("sqrt", x)


def rsqrt(x):
    return call("rsqrt", x)


def abs(x):  # noqa: A001
    return call("abs", x)


def tanh(x):
    return call("tanh", x)


def sigmoid(x):
    return call("sigmoid", x)


def print(*args, **kwargs):  # noqa: A001 - device printf is not traced
    return None


__all__ = [n for n in dir() if not n.startswith("_")]
