"""Match a traced prim_func to one of the operator families that have gfx950 kernels.

The reference lowers any TIR program through its PPL code generator (src/target/codegen_ppl.cc).
This build has hand-written kernels for a fixed set of families, so compilation is recognition: the op
trace is fingerprinted (which tile ops occur, how data flows from parameters through tiles), the
family's static parameters (shapes, dtypes, eps, scale, causal, page size, splits) are read out
of the program, and anything that does not fit a family is rejected with a clear error. There is
no generic code generation and no fallback.

Families and the reference programs they accept:
  rmsnorm  tpu_demo/rms_norm/rms_norm_fp16.py:9-35 (+ bf16 and fp32 twins, rmsnorm_fp32.py;
           optional weight parameter) and the split-K programs rmsnorm_splitk_{fp16,bf16,
           fp32}.py:9-47 (row sum accumulated over column blocks)
  gemm     tpu_demo/matmul/tpu_test_matmul_fp16.py:9-31 (+ bf16 / fp32-out variants, and
           tpu_test_matmul_fp32.py: fp32 A/B copied to fp16 tiles before ppl_gemm) and the
           fp8 programs examples/gemm_fp8/example_tilelang_gemm_fp8{,_2xAcc}.py
  rope     tpu_demo/tpu_test_rope_bf16.py:5-51 (4 params; fp16 / fp32 twins and tpu_test_rope.py)
           and a fused q+k form (6 params)
  swiglu   tpu_demo/tpu_test_swiglu_bf16.py:5-54 (+ tpu_test_swiglu_fp32.py)
  flashattn tpu_demo/flashattn/tpu_test_flashattn_bf16.py:14-135 (+ fp16, fp32 with fp16
           matrix tiles, and the all-fp32 tpu_demo/ppl/flashattn/fa_fp32.py) and the upstream
           examples/flash_attention/example_mha_fwd_bshd.py:30-151 structure, with grouped K/V heads (example_gqa_fwd_bshd.py:62-178), and the
           non-causal variable-length program example_mha_fwd_varlen.py:222-358
  sigmoid  tpu_demo/tpu_test_sigmoid_fp32.py:6-31 (ppl_sigmoid)
  gather   tpu_demo/tpu_test_gather_fp32.py:8-18 (ppl_gather)
  topk     tpu_demo/tpu_test_topk_fp32.py:6-18 (ppl_topk)
  row_reduce tpu_demo/tpu_test_reduce_max.py, tpu_test_reduce_sum.py
  elementwise tpu_demo/ppl/test/{exp,mul_N_1,elementwise_c}.py and tpu_demo/ppl/
           elementwise_add_kernel/elementwise_add.py: any chain of elementwise ppl ops between
           tile copies, evaluated into a register program
  mla      examples/deepseek_mla/example_mla_decode_paged.py:10-256 (split and no-split forms),
           with fp16/bf16 or fp8-e4m3 (+ fp32 scale parameter) KV; the non-paged
           examples/deepseek_mla/example_mla_decode.py:10-227 and the TPU program
           tpu_demo/ppl/deepseek_mla/mla_decode.py:9-121
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

from ....language import ir
from ....language.ir import Buffer, BufferAccess, Expr

LOG2E_REF = 1.44269504  # the constant the reference programs fold into exp2 scales


class UnsupportedProgram(ValueError):
    """The traced program matches no operator family implemented for gfx950."""


@dataclass
class Plan:
    family: str
    params: List[Buffer]
    out_idx: List[int]
    attrs: Dict = field(default_factory=dict)

    def describe(self) -> str:
        a = ", ".join(f"{k}={v}" for k, v in self.attrs.items())
        return f"{self.family}({a})"


# ------------------------------------------------------------------------------------------------
# trace helpers

_COPY = ("ppl_copy", "copy")
_GEMM = ("ppl_gemm", "gemm")
_STRUCTURAL = ("loop_begin", "loop_end", "alloc", "branch")


def _ops(pf, names=None):
    for op in pf.ops:
        if op.name in _STRUCTURAL:
            continue
        if names is None or op.name in names:
            yield op


def _buf(x) -> Optional[Buffer]:
    if isinstance(x, Buffer):
        return x
    if isinstance(x, BufferAccess):
        return x.buffer
    return None


def _op_names(pf):
    return [op.name for op in _ops(pf)]


def _source_param(pf, buf: Buffer, depth=0) -> Optional[Buffer]:
    """Follow tile copies (or element stores ``tile[i, j] = param[...]``) backwards from ``buf``
    to the global parameter it was loaded from."""
    if buf is None or depth > 8:
        return None
    if buf.scope == "global":
        return buf
    for op in _ops(pf, _COPY):
        if _buf(op.args[1]) is buf:
            src = _source_param(pf, _buf(op.args[0]), depth + 1)
            if src is not None:
                return src
    for op in _ops(pf, ("store",)):
        if op.args[0] is buf and isinstance(op.args[2], BufferAccess):
            src = _source_param(pf, op.args[2].buffer, depth + 1)
            if src is not None:
                return src
    return None


def _sink_param(pf, buf: Buffer, depth=0) -> Optional[Buffer]:
    """Follow tile copies forwards from ``buf`` to the global parameter it is stored to."""
    if buf is None or depth > 8:
        return None
    if buf.scope == "global":
        return buf
    for op in _ops(pf, _COPY):
        if _buf(op.args[0]) is buf:
            dst = _sink_param(pf, _buf(op.args[1]), depth + 1)
            if dst is not None:
                return dst
    for op in _ops(pf, ("store",)):
        v = op.args[2]
        if isinstance(v, BufferAccess) and v.buffer is buf:
            dst = _sink_param(pf, op.args[0], depth + 1)
            if dst is not None:
                return dst
    return None


def _written_params(pf):
    out = []
    for op in _ops(pf):
        b = None
        if op.name in _COPY:
            b = _buf(op.args[1])
        elif op.name == "store":
            b = op.args[0]
        if b is not None and b.scope == "global" and all(b is not o for o in out):
            out.append(b)
    return out


def _index(pf, buf) -> int:
    for i, p in enumerate(pf.params):
        if p is buf:
            return i
    raise UnsupportedProgram(f"{buf!r} is not a parameter")


def _symbolic(pf, gemms: Optional[List] = None):
    """The values a program stores, as expressions over its parameters: a list of
    (parameter index, expression) per store to a parameter, in program order, or None when the
    program uses an op outside the elementwise / row-reduce / rope vocabulary (or a gemm, when
    ``gemms`` is None; otherwise each gemm appends (op, ("gemm", a, b)) to it and its result
    tile takes that value).

    Tiles are followed through the program in order, so a tile written twice (``x = x * r``)
    carries its latest value. Expressions are tuples: ("load", i) for a tile copied from
    parameter i, ("const", v), (op, a, b) for add / sub / mul / div (operands of add and mul in a
    canonical order), ("add_C" / "mul_C", a, ("const", v)), ("exp", a), ("rsqrt", a),
    ("sigmoid", a), ("rsum", a) for a row sum and ("rope", e1, e2, o1, o2). Casts between tile
    dtypes and loop structure do not appear: a split-K accumulation ``acc = acc + rsum(x * x)``
    over a loop reads as one step from the filled accumulator. The dedicated families compare
    these expressions with the computation their kernel performs, and take their parameter
    roles from them rather than from parameter positions."""
    val: Dict[int, tuple] = {}
    stores: List[tuple] = []

    def get(b):
        b = _buf(b)
        return val.get(id(b), ("?",)) if b is not None else ("?",)

    def sym(op, a, b):
        if op in ("add", "mul") and repr(b) < repr(a):
            a, b = b, a
        return (op, a, b)

    for op in _ops(pf):
        n = op.name
        if n in _COPY:
            sb, db = _buf(op.args[0]), _buf(op.args[1])
            if sb is None or db is None:
                return None
            if sb.scope == "global" and db.scope == "global":
                return None
            if sb.scope == "global":
                val[id(db)] = ("load", _index(pf, sb))
            elif db.scope == "global":
                stores.append((_index(pf, db), get(sb)))
            else:
                val[id(db)] = get(sb)
        elif n in _FILL_OPS:
            val[id(_buf(op.args[0]))] = ("const", _const(op.args[1]))
        elif n in ("ppl_add", "ppl_sub", "ppl_mul", "ppl_div"):
            val[id(_buf(op.args[0]))] = sym(n[4:], get(op.args[1]), get(op.args[2]))
        elif n in ("ppl_add_C", "ppl_mul_C"):
            val[id(_buf(op.args[0]))] = (n[4:], get(op.args[1]), ("const", _const(op.args[2])))
        elif n == "ppl_exp":
            val[id(_buf(op.args[0]))] = ("exp", get(op.args[0]))
        elif n in ("ppl_rsqrt", "ppl_sigmoid"):
            val[id(_buf(op.args[0]))] = (n[4:], get(op.args[1]))
        elif n in ("ppl_reduce_sum", "ppl_reduce_max", "reduce_sum", "reduce_max"):
            if op.kwargs.get("dim", 1) not in (1, -1):
                return None
            r = ("rsum" if "sum" in n else "rmax", get(op.args[0]))
            if not op.kwargs.get("clear", True):  # accumulates into the output's contents
                r = ("acc_" + r[0], get(op.args[1]), r)
            val[id(_buf(op.args[1]))] = r
        elif n == "ppl_rope_add":
            val[id(_buf(op.args[0]))] = ("rope",) + tuple(get(a) for a in op.args[1:5])
        elif n in _GEMM and gemms is not None:
            r = ("gemm", get(op.args[0]), get(op.args[1]))
            gemms.append((op, r))
            val[id(_buf(op.args[2]))] = r
        else:
            return None
    return stores


def _neg(e) -> tuple:
    return ("mul_C", e, ("const", -1.0))


def _mul(a, b) -> tuple:
    return ("mul", a, b) if repr(a) <= repr(b) else ("mul", b, a)


def _add(a, b) -> tuple:
    return ("add", a, b) if repr(a) <= repr(b) else ("add", b, a)


def _shape(b: Buffer):
    return tuple(int(ir.const_value(s)) for s in b.shape)


def _const(x) -> float:
    if isinstance(x, Expr) and x.op == "const":
        return float(x.args[0])
    if isinstance(x, (int, float)):
        return float(x)
    raise UnsupportedProgram(f"expected a compile-time constant, got {x!r}")


def _fail(family, msg):
    raise UnsupportedProgram(f"{family}: {msg}")


# Tile ops each family's kernel implements. A program that issues any other op (an epilogue, a
# bias add, a scale) computes something the kernel does not, and is rejected.
_FILL_OPS = ("ppl_fill", "fill")
_ALLOWED_OPS = {
    "rmsnorm": _COPY + _FILL_OPS + ("ppl_reduce_sum", "ppl_mul", "ppl_add", "ppl_add_C",
                                    "ppl_mul_C", "ppl_rsqrt"),
    "gemm": _COPY + _FILL_OPS + _GEMM + ("store",),
    "rope": _COPY + ("ppl_mul", "ppl_mul_C", "ppl_rope_add"),
    "swiglu": _COPY + _FILL_OPS + ("ppl_exp", "ppl_mul_C", "ppl_add", "ppl_div", "ppl_mul"),
    "flashattn": _COPY + _FILL_OPS + _GEMM + ("store", "ppl_add", "ppl_sub", "ppl_mul",
                                              "ppl_div", "ppl_exp", "ppl_mul_C", "ppl_reduce_max",
                                              "ppl_reduce_sum", "reduce_max", "reduce_sum"),
    "mla": _COPY + _FILL_OPS + _GEMM + ("store", "reduce_max", "reduce_sum", "ppl_add",
                                        "ppl_sub", "ppl_mul", "ppl_div", "ppl_exp", "ppl_mul_C",
                                        "ppl_reduce_max", "ppl_reduce_sum"),
    "sigmoid": _COPY + ("ppl_sigmoid",),
    "gather": ("ppl_gather",),
    "topk": ("ppl_topk",),
    "row_reduce": _COPY + _FILL_OPS + ("ppl_reduce_max", "ppl_reduce_sum", "reduce_max",
                                       "reduce_sum"),
    "elementwise": _COPY + _FILL_OPS + ("ppl_add", "ppl_sub", "ppl_mul", "ppl_div", "ppl_add_C",
                                        "ppl_mul_C", "ppl_exp", "ppl_rsqrt", "ppl_sigmoid"),
    "mlp": _COPY + _FILL_OPS + _GEMM + ("ppl_exp", "ppl_mul_C", "ppl_add", "ppl_div", "ppl_mul"),
}


def _audit(pf, plan: "Plan", used: Optional[List] = None) -> "Plan":
    """Reject a matched program that issues an op outside its family's kernel or has a
    parameter the kernel never reads or writes. ``used`` lists the parameters the matched
    pattern consumed (default: every integer-valued attr that indexes ``pf.params``)."""
    fam = plan.family
    extra = sorted({op.name for op in _ops(pf)} - set(_ALLOWED_OPS[fam]))
    if extra:
        _fail(fam, f"op(s) {extra} are not part of the {fam} kernel (an epilogue or extra "
                   f"elementwise step would be dropped), so the program is not compiled")
    if used is None:
        idx = {plan.attrs[k] for k in _PARAM_ATTRS[fam] if plan.attrs.get(k) is not None}
        if fam == "elementwise":
            idx = set(plan.attrs["inputs"]) | set(plan.attrs["outputs"])
        used = [pf.params[i] for i in sorted(idx)]
    unused = [getattr(p, "name", repr(p)) for p in pf.params if all(p is not u for u in used)]
    if unused:
        _fail(fam, f"parameter(s) {unused} are not read or written by the {fam} kernel")
    return plan


# plan attrs that hold parameter indices, per family
_PARAM_ATTRS = {
    "rmsnorm": ("x", "w", "y"),
    "gemm": ("a", "b", "c"),
    "rope": ("q", "k", "cos", "sin", "q_out", "k_out"),
    "swiglu": ("gate", "up", "out"),
    "flashattn": ("q", "k", "v", "o", "cu_q", "cu_k", "max_q", "glse", "partial"),
    "mla": ("q", "q_pe", "kv", "k_pe", "block_table", "seqlens", "o", "glse", "o_partial",
            "kv_scale"),
    "sigmoid": ("x", "y"),
    "gather": ("param", "index", "out"),
    "topk": ("src", "values", "indices"),
    "row_reduce": ("x", "y"),
    "elementwise": (),
    "mlp": ("x", "wg", "wu", "wd", "out"),
}


# ------------------------------------------------------------------------------------------------
# families


def _rmsnorm(pf, names) -> Plan:
    fam = "rmsnorm"
    red = [op for op in _ops(pf, ("ppl_reduce_sum",))]
    if len(red) != 1 or red[0].kwargs.get("dim", 1) not in (1, -1):
        _fail(fam, "expected one row reduce_sum over the last dim")
    acc = _buf(red[0].args[1])
    sq = _buf(red[0].args[0])
    # split-K programs add each block's row sum into a running sum: follow that accumulation
    for op in _ops(pf, ("ppl_add",)):
        srcs = (_buf(op.args[1]), _buf(op.args[2]))
        dst = _buf(op.args[0])
        if acc in srcs and dst is not acc and dst in srcs:
            acc = dst
            break
    # eps and 1/N applied to the reduced buffer
    eps = None
    inv = None
    for op in _ops(pf, ("ppl_add_C", "ppl_mul_C")):
        if _buf(op.args[1]) is acc:
            if op.name == "ppl_add_C":
                eps = _const(op.args[2])
            else:
                inv = _const(op.args[2])
    if eps is None or inv is None:
        _fail(fam, "could not read eps / 1/N from ppl_add_C / ppl_mul_C on the row sum")
    # x is what the squared tile was computed from
    mul = [op for op in _ops(pf, ("ppl_mul",)) if _buf(op.args[0]) is sq]
    if not mul:
        _fail(fam, "no x*x feeding the reduction")
    x = _source_param(pf, _buf(mul[0].args[1]))
    writes = _written_params(pf)
    if x is None or len(writes) != 1:
        _fail(fam, "expected one input x and one output y")
    y = writes[0]
    if len(x.shape) < 2 or _shape(x) != _shape(y) or x.dtype != y.dtype:
        _fail(fam, f"x {x!r} and y {y!r} must match")
    N = _shape(x)[-1]
    if abs(inv * N - 1.0) > 1e-6:
        _fail(fam, f"mean scale {inv} is not 1/{N}")
    if x.dtype not in ("float16", "bfloat16", "float32"):
        _fail(fam, f"dtype {x.dtype} (float16 / bfloat16 / float32 kernels only)")
    w = None
    for p in pf.params:
        if p is x or p is y:
            continue
        if math.prod(_shape(p)) == N and p.dtype == x.dtype:
            w = p
        else:
            _fail(fam, f"unexpected parameter {p!r}")
    # the stored value, as the program computes it: x * rsqrt(rowsum(x * x) * inv + eps),
    # times w when there is a weight (the row sum optionally accumulated into a zero-filled sum)
    X = ("load", _index(pf, x))
    S = ("rsum", _mul(X, X))
    R = [("rsqrt", ("add_C", ("mul_C", s_, ("const", inv)), ("const", eps)))
         for s_ in (S, _add(("const", 0.0), S))]
    want = [sorted(map(repr, [X, r] + ([] if w is None else [("load", _index(pf, w))])))
            for r in R]
    stores = _symbolic(pf)

    def factors(e):
        return factors(e[1]) + factors(e[2]) if e[0] == "mul" else [e]

    if not stores or any(o != _index(pf, y) or sorted(map(repr, factors(e))) not in want
                         for o, e in stores):
        _fail(fam, "the stored value is not x * rsqrt(mean(x * x) + eps)" +
              ("" if w is None else " * w"))
    # whole rows: every copy of x and every store to y spans the row (one tile, or column
    # tiles stepped by a loop), all at one row-tile position; a row sum taken inside a loop is
    # accumulated into a sum filled outside it (else only the last column tile would count)
    rows = []
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        for g, t in ((src, db), (dst, sb)):
            gb = _buf(g)
            if gb is x or gb is y:
                if t.scope == "global" or not _covers_rows(op, g, t, N):
                    _fail(fam, f"a tile copy of {gb!r} does not span whole rows")
                rows.append(_tile_map(pf, g, t, skip=-1))
    if not rows or rows[0] is None or any(r != rows[0] for r in rows):
        _fail(fam, "the tile copies of x and y are not at one row-tile position")
    if red[0].loops:
        fills = [op for op in _ops(pf, _FILL_OPS) if _buf(op.args[0]) is acc]
        if len(fills) != 1 or any(lp in (fills[0].loops or ()) for lp in red[0].loops):
            _fail(fam, "a row sum inside a loop must accumulate into a sum cleared outside it")
    outs = [_index(pf, y)]
    return Plan(fam, pf.params, outs, dict(
        x=_index(pf, x), w=None if w is None else _index(pf, w), y=outs[0], eps=eps,
        rows=math.prod(_shape(x)[:-1]), cols=N, dtype=x.dtype))


def _swiglu(pf, names) -> Plan:
    """out = up * (gate / (exp(-gate) + 1)) (tpu_test_swiglu_bf16.py:41-49), with the roles of
    gate and up read from the stored expression. Another expression is not this kernel's (the
    caller then tries the general elementwise program)."""
    fam = "swiglu"
    stores = _symbolic(pf)
    if not stores or len(stores) != 1:
        _fail(fam, "expected one stored tile")
    o, e = stores[0]
    gate = up = None
    if e[0] == "mul":
        for u, q in ((e[1], e[2]), (e[2], e[1])):
            if u[0] == "load" and q[0] == "div" and q[1][0] == "load" and q[1] != u and \
                    q == ("div", q[1], _add(("exp", _neg(q[1])), ("const", 1.0))):
                gate, up = q[1][1], u[1]
    if gate is None:
        _fail(fam, "the stored tile is not up * (gate / (exp(-gate) + 1))")
    P = pf.params
    gate, up, out = P[gate], P[up], P[o]
    if len(P) != 3:
        _fail(fam, "expected (gate, up) -> out")
    if not (_shape(gate) == _shape(up) == _shape(out)):
        _fail(fam, "gate, up, out shapes differ")
    if not (gate.dtype == up.dtype == out.dtype) or gate.dtype not in ("bfloat16", "float16",
                                                                       "float32"):
        _fail(fam, "dtypes must all be bfloat16, all float16 or all float32")
    maps = []
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        if sb is not None and db is not None and (sb.scope == "global") != (db.scope == "global"):
            maps.append(_tile_map(pf, src, db) if sb.scope == "global" else
                        _tile_map(pf, dst, sb))
    if not maps or maps[0] is None or any(m != maps[0] for m in maps):
        _fail(fam, "the tile copies of gate, up and out are not at one grid position")
    return Plan(fam, P, [_index(pf, out)], dict(
        gate=_index(pf, gate), up=_index(pf, up), out=_index(pf, out),
        n=math.prod(_shape(gate)), dtype=gate.dtype))


def _rope_term(e1, e2, o1, o2):
    """(x, cos, sin) parameter indices when the ppl_rope_add operands are the demo's tiles
    x*cos, -(x*sin), x*cos, x*sin (tpu_test_rope_bf16.py:28-45) of three distinct parameters,
    else None. The negation may sit on the product, on x or on sin."""
    if e1 != o1 or e1[0] != "mul" or o2[0] != "mul":
        return None
    a, b, c, d = e1[1], e1[2], o2[1], o2[2]
    if any(t[0] != "load" for t in (a, b, c, d)):
        return None
    common = {a, b} & {c, d}
    if len(common) != 1:
        return None
    x = common.pop()
    cos = b if a == x else a
    sin = d if c == x else c
    if len({x, cos, sin}) != 3:
        return None
    if e2 not in (_neg(o2), _mul(_neg(x), sin), _mul(x, _neg(sin))):
        return None
    return x[1], cos[1], sin[1]


def _rope(pf, names) -> Plan:
    """Parameter roles come from the data flow into ppl_rope_add, not from positions: the
    reference's ppl/rope programs take (G_out, G_in, G_cos, G_sin), the tpu_test_rope demos
    (G_in, G_cos, G_sin, G_out)."""
    fam = "rope"
    stores = _symbolic(pf)
    if not stores or len(stores) > 2:
        _fail(fam, "expected one stored rope tile (x) or two (q and k)")
    terms = []
    for o, e in stores:
        t = _rope_term(*e[1:]) if e[0] == "rope" else None
        if t is None:
            _fail(fam, "the stored tile is not ppl_rope_add(out, x*cos, -x*sin, x*cos, x*sin) of "
                       "one input and one cos / sin table pair")
        terms.append(t + (o,))
    P = pf.params
    # every global tile copy must address the output tile's grid position (tables without the
    # head dimension of a 3-D q / k)
    maps: Dict[int, list] = {}
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        if sb is None or db is None:
            _fail(fam, "copy operands must be buffers")
        if sb.scope == "global" and db.scope != "global":
            maps.setdefault(_index(pf, sb), []).append(_tile_map(pf, src, db))
        elif db.scope == "global" and sb.scope != "global":
            maps.setdefault(_index(pf, db), []).append(_tile_map(pf, dst, sb))

    def same_position(x, c, s, o):
        mo = maps.get(o, [None])
        if len(mo) != 1 or mo[0] is None:
            return False
        mo = mo[0]
        tab = mo if len(mo) == 2 else [mo[0], mo[-1]]
        return all(m == mo for m in maps.get(x, [None])) and \
            all(m == tab for m in maps.get(c, [None]) + maps.get(s, [None]))

    if len(terms) == 1:
        x, c, s, o = terms[0]
        if len(P) != 4:
            _fail(fam, "the one-tensor form takes x, cos, sin and out (4 parameters)")
        if not (_shape(P[x]) == _shape(P[c]) == _shape(P[s]) == _shape(P[o])) or \
                len(_shape(P[x])) != 2:
            _fail(fam, "the 4-parameter form takes x, cos, sin, out of one [C, W] shape")
        C, W = _shape(P[x])
        attrs = dict(q=x, k=None, cos=c, sin=s, q_out=o, k_out=None, tokens=C, heads_q=1,
                     heads_k=0, dim=W)
        outs = [o]
    else:
        (xq, c, s, oq), (xk, c2, s2, ok) = terms
        if (c, s) != (c2, s2) or xq == xk or oq == ok or len(P) != 6:
            _fail(fam, "the q+k form rotates two inputs into two outputs with one table pair "
                       "(6 parameters)")
        if _shape(P[c]) != _shape(P[s]) or len(_shape(P[c])) != 2:
            _fail(fam, "cos/sin must be [tokens, dim]")
        T_, W = _shape(P[c])
        for xi, oi in ((xq, oq), (xk, ok)):
            xs = _shape(P[xi])
            if len(xs) < 2 or xs[0] != T_ or xs[-1] != W or _shape(P[oi]) != xs:
                _fail(fam, "q/k must be [tokens, heads, dim] matching the tables and outputs")
        attrs = dict(q=xq, k=xk, cos=c, sin=s, q_out=oq, k_out=ok, tokens=T_,
                     heads_q=math.prod(_shape(P[xq])[1:-1]),
                     heads_k=math.prod(_shape(P[xk])[1:-1]), dim=W)
        outs = sorted((oq, ok))
    for x, c, s, o in terms:
        if not same_position(x, c, s, o):
            _fail(fam, f"the tile copies of {P[x]!r}, its tables and {P[o]!r} are not at one "
                       f"grid position")
    dts = {p.dtype for p in P}
    if len(dts) != 1 or next(iter(dts)) not in ("bfloat16", "float16", "float32"):
        _fail(fam, f"all parameters must share one of bfloat16 / float16 / float32, got {dts}")
    if attrs["dim"] % 2:
        _fail(fam, "dim must be even")
    attrs["dtype"] = next(iter(dts))
    return Plan(fam, P, outs, attrs)


def _gemm(pf, names) -> Plan:
    fam = "gemm"
    g = list(_ops(pf, _GEMM))
    if len(g) != 1:
        _fail(fam, "expected one gemm")
    ta, tb = g[0].kwargs.get("transpose_A", False), g[0].kwargs.get("transpose_B", False)
    if ta:
        _fail(fam, "transpose_A is not supported")
    A = _source_param(pf, _buf(g[0].args[0]))
    B = _source_param(pf, _buf(g[0].args[1]))
    acc = _buf(g[0].args[2])
    C = _sink_param(pf, acc)
    if C is None:
        # the accumulator folded into a second fragment by element stores before the copy-out
        # (examples/gemm_fp8/example_tilelang_gemm_fp8_2xAcc.py:36-44)
        for op in _ops(pf, ("store",)):
            v = op.args[2]
            if isinstance(v, Expr) and any(e.op == "load" and e.args[0] is acc for e in v.walk()):
                C = _sink_param(pf, op.args[0])
                if C is not None:
                    break
    if A is None or B is None or C is None:
        _fail(fam, "could not trace A, B and C through the tile copies")
    M, K = _shape(A)
    if tb:
        N, Kb = _shape(B)
    else:
        Kb, N = _shape(B)
    if Kb != K or _shape(C) != (M, N):
        _fail(fam, f"shapes A{_shape(A)} B{_shape(B)} C{_shape(C)} do not chain")
    # dtype of the tiles the gemm multiplies (fp32 programs copy their tiles to fp16 first)
    ta_dt, tb_dt = _buf(g[0].args[0]).dtype, _buf(g[0].args[1]).dtype
    fp8 = ("float8_e4m3", "float8_e5m2")
    if ta_dt != tb_dt or ta_dt not in ("float16", "bfloat16") + fp8:
        _fail(fam, f"matrix tiles must be float16, bfloat16 or fp8 pairs (got {ta_dt}, {tb_dt})")
    if A.dtype != B.dtype or A.dtype not in ("float16", "bfloat16", "float32") + fp8:
        _fail(fam, "A and B must share a dtype: float16, bfloat16, fp8, or float32 cast to the "
                   "tiles")
    if A.dtype != "float32" and A.dtype != ta_dt:
        _fail(fam, f"A is {A.dtype} but the gemm multiplies {ta_dt} tiles")
    if A.dtype in fp8 and C.dtype not in ("float16", "bfloat16", "float32", A.dtype):
        _fail(fam, f"fp8 GEMM output {C.dtype} (float32, float16, bfloat16 or {A.dtype})")
    if A.dtype not in fp8 and C.dtype not in ("float16", "bfloat16", "float32"):
        _fail(fam, f"C dtype {C.dtype}")
    # the accumulator starts at zero (ppl_gemm accumulates into C) and the only element stores
    # allowed are the 2xAcc fold acc2[i, j] = acc2[i, j] + acc[i, j] of two local fragments
    for op in _ops(pf, _FILL_OPS):
        if _const(op.args[1]) != 0.0:
            _fail(fam, f"{op.name} of {_buf(op.args[0])!r} with {op.args[1]!r}: the kernel's "
                       "accumulators start at zero")
    for op in _ops(pf, ("store",)):
        v = op.args[2]
        nodes = list(v.walk()) if isinstance(v, Expr) else [v]
        loads = [e for e in nodes if isinstance(e, Expr) and e.op == "load"]
        other = [e for e in nodes if not (isinstance(e, Expr) and e.op in ("load", "add"))
                 and not isinstance(e, (BufferAccess, ir.Var))]
        if op.args[0].scope == "global" or other or len(loads) != 2 or \
                any(e.args[0].scope == "global" for e in loads) or \
                all(e.args[0] is not op.args[0] for e in loads):
            _fail(fam, f"element store into {op.args[0]!r} is not the accumulator fold "
                       "acc2[i, j] += acc[i, j]; epilogues are not part of the gemm kernel")
    # The tiles multiplied are the kernel's: A's row tile and B's column tile at C's tile
    # position, both stepped over all of K by the loop around the gemm, into an accumulator
    # cleared before that loop. (A clear inside it keeps only the tiles after the last clear,
    # unless a fold into a second accumulator precedes it, and that fold must run on the last
    # k tile: example_tilelang_gemm_fp8_2xAcc.py:36-44 folds every 128 / block_K tiles.)
    kd_b = 1 if tb else 0
    cmap = None
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        if db is C and sb.scope != "global":
            cmap = _tile_map(pf, dst, sb)
    if cmap is None:
        _fail(fam, "C is not stored as one tile of a grid covering it")
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        if db.scope == "global" or sb not in (A, B) or (sb is A and sb is B):
            continue
        kd = 1 if sb is A else kd_b
        m = _tile_map(pf, src, db, skip=kd)
        if m is None or not _covers_rows(op, src, db, K, d=kd) or \
                m[1 - kd] != (cmap[0] if sb is A else cmap[1]):
            _fail(fam, f"the tile copies of {sb!r} do not step over all of K at C's tile "
                       "position")
    loops = g[0].loops or ()
    folded = any(op.name == "store" for op in _ops(pf))
    for op in _ops(pf, _FILL_OPS):
        if _buf(op.args[0]) is acc and any(lp in (op.loops or ()) for lp in loops) and not folded:
            _fail(fam, "the accumulator is cleared inside the k loop")
    if loops:
        names, last = [], {}
        for lp in loops:
            for v, ext in zip(lp.vars, lp.extents):
                n = _extent_value(ext)
                if n is None or not isinstance(v, Expr):
                    _fail(fam, "k loop without a static extent")
                last[v.args[0]] = n - 1
        for op in pf.ops:
            if op.name == "branch" and any(lp in (op.loops or ()) for lp in loops):
                if not _eval_env(op.args[0], last):
                    _fail(fam, "a branch inside the k loop is not taken on the last k tile, so "
                               "the program leaves its last tiles out of C")
    return Plan(fam, pf.params, [_index(pf, C)], dict(
        a=_index(pf, A), b=_index(pf, B), c=_index(pf, C), M=M, N=N, K=K, trans_b=bool(tb),
        in_dtype=A.dtype, out_dtype=C.dtype,
        operand_dtype=ta_dt if A.dtype == "float32" else None))


def _pipelined_extents(pf):
    return [op.args[0].extents[0] for op in pf.ops
            if op.name == "loop_begin" and op.args[0].kind == "pipelined"]


def _flashattn(pf, names) -> Plan:
    fam = "flashattn"
    g = list(_ops(pf, _GEMM))
    qk = [op for op in g if op.kwargs.get("transpose_B")]
    pv = [op for op in g if not op.kwargs.get("transpose_B")]
    if len(qk) != 1 or len(pv) != 1:
        _fail(fam, "expected Q@K^T and P@V")
    Q = _source_param(pf, _buf(qk[0].args[0]))
    K = _source_param(pf, _buf(qk[0].args[1]))
    V = _source_param(pf, _buf(pv[0].args[1]))
    acc_o = _buf(pv[0].args[2])
    O = _sink_param(pf, acc_o)
    if None in (Q, K, V, O):
        _fail(fam, "could not trace Q, K, V and Output")
    shp = _shape(Q)
    kshp = _shape(K)
    if len(shp) == 3:
        return _flashattn_varlen(pf, qk[0], pv[0], Q, K, V, O)
    if len(_shape(O)) == 5:
        return _flashattn_splitkv(pf, qk[0], pv[0], Q, K, V, O)
    bhsd = _seq_dim(pf, Q) == 2
    if bhsd:
        if len(shp) != 4 or shp != _shape(O) or kshp != _shape(V) or len(kshp) != 4:
            _fail(fam, "Q, Output must be [batch, heads, seq_q, dim] and K, V "
                       "[batch, kv_heads, seq_kv, dim]")
        if (kshp[0], kshp[3]) != (shp[0], shp[3]) or shp[1] % kshp[1]:
            _fail(fam, f"K/V {kshp} do not group Q {shp} (query heads a multiple of K/V heads)")
    else:
        if len(shp) != 4 or shp != _shape(O) or kshp != _shape(V) or len(kshp) != 4:
            _fail(fam, "Q, Output must be [batch, seq, heads, dim] and K, V "
                       "[batch, seq, kv_heads, dim]")
        if (kshp[0], kshp[1], kshp[3]) != (shp[0], shp[1], shp[3]) or shp[2] % kshp[2]:
            _fail(fam, f"K/V {kshp} do not group Q {shp} (query heads a multiple of K/V heads)")
    # tiles the two gemms multiply: the fp32 program copies Q, K, V and P to fp16 tiles first
    tile_dts = {_buf(qk[0].args[0]).dtype, _buf(qk[0].args[1]).dtype, _buf(pv[0].args[0]).dtype,
                _buf(pv[0].args[1]).dtype}
    if len(tile_dts) != 1 or next(iter(tile_dts)) not in ("bfloat16", "float16", "float32"):
        _fail(fam, f"the gemm tiles must all be bfloat16, all float16 or all float32, got "
                   f"{tile_dts}")
    tile_dt = next(iter(tile_dts))
    if tile_dt == "float32" and not (Q.dtype == K.dtype == V.dtype == O.dtype == "float32"):
        _fail(fam, "fp32 gemm tiles need fp32 Q, K, V and Output")
    if not (Q.dtype == K.dtype == V.dtype == O.dtype):
        _fail(fam, "Q, K, V and Output must share a dtype")
    if Q.dtype not in (tile_dt, "float32"):
        _fail(fam, f"parameters are {Q.dtype} but the gemms multiply {tile_dt} tiles")
    if bhsd and Q.dtype == "float32":
        _fail(fam, "head-major programs take bfloat16 or float16 parameters")
    B, S, H, D = (shp[0], shp[2], shp[1], shp[3]) if bhsd else shp
    # causal: the KV loop is truncated at the diagonal (T.min(...) in the extent), or scores
    # are masked by comparing query and key positions.
    causal = any(isinstance(e, Expr) and e.has_op("min") for e in _pipelined_extents(pf))
    for op in _ops(pf, ("store",)):
        v = op.args[2]
        if isinstance(v, Expr) and v.has_op("if_then_else"):
            for e in v.walk():
                if e.op == "if_then_else" and isinstance(e.args[0], Expr):
                    fv = e.args[0].free_vars()
                    if any(n.startswith("bx") for n in fv):
                        causal = True
    # softmax scale
    acc_s = _buf(qk[0].args[2])
    if "ppl_exp" in names:
        cands = [op for op in _ops(pf, ("ppl_mul_C",)) if _buf(op.args[0]) is acc_s]
        if not cands:
            _fail(fam, "no ppl_mul_C scaling the scores")
        sm_scale = _const(cands[0].args[2])
    else:
        sm_scale = None
        for op in _ops(pf, ("store",)):
            if op.args[0] is acc_s and isinstance(op.args[2], Expr) and op.args[2].has_op("exp2"):
                cs = [c for c in op.args[2].consts() if isinstance(c, float) and c > 0]
                if cs:
                    sm_scale = cs[0] / LOG2E_REF
        if sm_scale is None:
            _fail(fam, "could not read the softmax scale")
    # Output's tile is stored where Q's tile was read, and without a causal bound the K and V
    # tiles step over every key
    qm = om = None
    seqd = 2 if bhsd else 1
    for op in _ops(pf, _COPY):
        src, dst = op.args[0], op.args[1]
        sb, db = _buf(src), _buf(dst)
        if sb is Q and db.scope != "global":
            qm = _tile_map(pf, src, db)
        elif db is O and sb.scope != "global":
            om = _tile_map(pf, dst, sb)
        elif sb in (K, V) and db.scope != "global" and not causal and \
                not _covers_rows(op, src, db, kshp[seqd], d=seqd):
            _fail(fam, f"the tile copies of {sb!r} do not step over every key")
    if qm is None or qm != om:
        _fail(fam, "Output's tile is not stored at the position its Q tile was read from")
    if bhsd:
        # example_mha_fwd_bhsd.py:50-55 masks with q_idx = bx * block_M + i + seq_kv - seq_q
        # while its loop bound (:139-141) stops at key (bx + 1) * block_M and its reference
        # (:183) uses the top-left torch.tril: the three agree only when seq_q == seq_kv.
        if causal and S != kshp[2]:
            _fail(fam, f"causal with seq_q {S} != seq_kv {kshp[2]}: the example's mask, loop "
                       "bound and reference disagree there")
        return Plan(fam, pf.params, [_index(pf, O)], dict(
            q=_index(pf, Q), k=_index(pf, K), v=_index(pf, V), o=_index(pf, O), B=B, S=S,
            S_kv=kshp[2], H=H, H_kv=kshp[1], D=D, causal=causal, sm_scale=sm_scale,
            dtype=Q.dtype, operand_dtype=None, layout="bhsd"))
    return Plan(fam, pf.params, [_index(pf, O)], dict(
        q=_index(pf, Q), k=_index(pf, K), v=_index(pf, V), o=_index(pf, O), B=B, S=S, H=H,
        H_kv=kshp[2], D=D,
        causal=causal, sm_scale=sm_scale, dtype=Q.dtype,
        operand_dtype=tile_dt if Q.dtype == "float32" and tile_dt != "float32" else None))


def _flashattn_splitkv(pf, qk, pv, Q, K, V, Opart) -> Plan:
    """examples/flash_attention/example_mha_inference.py:98-203: the query block's online softmax
    over each of num_split key ranges (flash_attn_split) writes normalised partial outputs to
    Output_partial [batch, seq_q, heads, num_split, dim] and log2 sum-exp to glse [batch, heads,
    num_split, seq_q]; combine merges them into Output [batch, seq_q, heads, dim]. The merge of
    the splits equals attention over all keys when every split covers whole key tiles. The
    program's partials (each split's normalised output and log2 sum-exp, in the program's
    dtype) are written as the program writes them, and Output is their combine."""
    fam = "flashattn"
    shp, kshp, pshp = _shape(Q), _shape(K), _shape(Opart)
    if len(shp) != 4 or len(kshp) != 4 or kshp != _shape(V):
        _fail(fam, "split-KV Q must be [batch, seq_q, heads, dim] and K, V [batch, seq_kv, heads, "
                   "dim]")
    B, Sq, H, D = shp
    Skv, Hkv = kshp[1], kshp[2]
    if (kshp[0], kshp[3]) != (B, D) or Hkv == 0 or H % Hkv:
        _fail(fam, f"K/V {kshp} do not match Q {shp}")
    if len(pshp) != 5 or (pshp[0], pshp[1], pshp[2], pshp[4]) != (B, Sq, H, D):
        _fail(fam, f"Output_partial {pshp} is not [batch, seq_q, heads, num_split, dim]")
    ns = pshp[3]
    outs = [p for p in pf.params if isinstance(p, Buffer) and p not in (Q, K, V, Opart) and
            _shape(p) == shp]
    lses = [p for p in pf.params if isinstance(p, Buffer) and list(_shape(p)) == [B, H, ns, Sq]]
    if len(outs) != 1 or len(lses) != 1 or len(pf.kernels) != 2:
        _fail(fam, "split-KV attention needs glse [batch, heads, num_split, seq_q], "
                   "Output_partial and one Output [batch, seq_q, heads, dim] written by a second "
                   "(combine) kernel")
    O = outs[0]
    if not (Q.dtype == K.dtype == V.dtype == O.dtype == lses[0].dtype == Opart.dtype) or \
            Q.dtype not in ("bfloat16", "float16"):
        _fail(fam, "split-KV attention takes one bfloat16 or float16 dtype for Q, K, V, glse, "
                   "Output_partial and Output")
    if ns > 16:
        _fail(fam, f"{ns} splits (at most 16)")
    tile_dts = {_buf(qk.args[0]).dtype, _buf(qk.args[1]).dtype, _buf(pv.args[0]).dtype,
                _buf(pv.args[1]).dtype}
    if tile_dts != {Q.dtype}:
        _fail(fam, f"the gemms multiply {tile_dts} tiles of {Q.dtype} parameters")
    block_N = _shape(_buf(qk.args[1]))[0]
    if Skv % ns or (Skv // ns) % block_N:
        _fail(fam, f"seq_kv {Skv} does not split into {ns} ranges of whole {block_N}-key tiles "
                   "(the program would drop or overlap keys there)")
    if any(isinstance(e, Expr) and e.has_op("min") for e in _pipelined_extents(pf)):
        _fail(fam, "the split program's causal form (loop bound without the split offset) is not "
                   "causal attention")
    acc_s = _buf(qk.args[2])
    sm_scale = None
    for op in _ops(pf, ("store",)):
        if op.args[0] is acc_s and isinstance(op.args[2], Expr) and op.args[2].has_op("exp2"):
            cs = [c for c in op.args[2].consts() if isinstance(c, float) and c > 0]
            if cs:
                sm_scale = cs[0] / LOG2E_REF
    if sm_scale is None:
        _fail(fam, "could not read the softmax scale")
    return Plan(fam, pf.params, [_index(pf, O)], dict(
        q=_index(pf, Q), k=_index(pf, K), v=_index(pf, V), o=_index(pf, O), B=B, S=Sq, S_kv=Skv,
        H=H, H_kv=Hkv, D=D, causal=False, sm_scale=sm_scale, dtype=Q.dtype, operand_dtype=None,
        layout="bshd_kv", num_split=ns, glse=_index(pf, lses[0]), partial=_index(pf, Opart)))


def _mlp(pf, names) -> Plan:
    """tpu_demo/ppl/mlp/mlp_bf16.py:10-141 and mlp_fp32.py:7-120 (DeepSeek-V3 MLP; the fp32
    program copies its fp32 tiles to bf16 tiles for the gemms): gate / up projections
    x W^T (ppl_gemm transpose_B into 16-bit tiles), SiLU(gate) * up in fp32 rounded once to
    the 16-bit type, down projection gated Wd^T. Every workgroup reduces over one hidden block
    and one intermediate block and overwrites its output block, so the program is the MLP only
    when those blocks are whole (Block_h = hidden_size, Block_i = intermediate_size); other
    blockings store a partial, order-dependent result that is not compiled."""
    fam = "mlp"
    g = list(_ops(pf, _GEMM))
    if len(g) != 3 or not all(op.kwargs.get("transpose_B") for op in g):
        _fail(fam, "expected three ppl_gemm with transpose_B (gate, up, down)")
    a = [_buf(op.args[0]) for op in g]
    shared = [(i, j) for i in range(3) for j in range(i + 1, 3) if a[i] is a[j]]
    if len(shared) != 1:
        _fail(fam, "gate and up projections must multiply the same x tile")
    i, j = shared[0]
    down = g[3 - i - j]
    divs = list(_ops(pf, ("ppl_div",)))
    if len(divs) != 1:
        _fail(fam, "expected one ppl_div (SiLU)")
    num = _buf(divs[0].args[1])  # SiLU numerator: the fp32 copy of the gate tile

    def feeds(tile, target):
        return any(_buf(op.args[0]) is tile and _buf(op.args[1]) is target
                   for op in _ops(pf, _COPY)) or tile is target
    gate = [op for op in (g[i], g[j]) if feeds(_buf(op.args[2]), num)]
    if len(gate) != 1:
        _fail(fam, "could not tell the gate projection (the SiLU input) from the up projection")
    gate = gate[0]
    up = g[i] if gate is g[j] else g[j]
    x = _source_param(pf, a[i])
    wg, wu = _source_param(pf, _buf(gate.args[1])), _source_param(pf, _buf(up.args[1]))
    wd = _source_param(pf, _buf(down.args[1]))
    out = _sink_param(pf, _buf(down.args[2]))
    if None in (x, wg, wu, wd, out) or len({id(p) for p in (x, wg, wu, wd, out)}) != 5:
        _fail(fam, "could not trace x, gate_weight, up_weight, down_weight and output")
    M, Hd = _shape(x)
    I = _shape(wg)[0]
    if list(_shape(out)) != [M, Hd] or list(_shape(wg)) != [I, Hd] or \
            list(_shape(wu)) != [I, Hd] or list(_shape(wd)) != [Hd, I]:
        _fail(fam, "shapes must be x, output [rows, hidden], gate / up weights [inter, hidden], "
                   "down weight [hidden, inter]")
    dt = x.dtype
    if dt not in ("bfloat16", "float16", "float32") or \
            any(p.dtype != dt for p in (wg, wu, wd, out)):
        _fail(fam, "parameters must all be bfloat16, all float16 or all float32")
    # the projections multiply and store 16-bit tiles: of the parameter dtype, or (all-fp32
    # program, tpu_demo/ppl/mlp/mlp_fp32.py) of one 16-bit operand dtype the fp32 tiles are
    # copied to
    tdt = {_buf(op.args[k]).dtype for op in g for k in range(3)}
    if len(tdt) != 1 or (dt != "float32" and tdt != {dt}) or \
            not tdt <= {"bfloat16", "float16"}:
        _fail(fam, "the projections must multiply and store 16-bit tiles of one dtype (the "
                   "parameter dtype for 16-bit parameters)")
    operand = next(iter(tdt)) if dt == "float32" else None
    # what the down projection multiplies and what is stored: up * (gate / (exp(-gate) + 1))
    # of the two projections of x, and the down projection of it
    recs: List[tuple] = []
    stores = _symbolic(pf, recs)
    ex = {id(op): r for op, r in recs}
    G, U, D = ex.get(id(gate)), ex.get(id(up)), ex.get(id(down))
    if stores is None or None in (G, U, D) or \
            D[1] != _mul(U, ("div", G, _add(("exp", _neg(G)), ("const", 1.0)))) or \
            stores != [(_index(pf, out), D)] or G[1] != ("load", _index(pf, x)) or \
            U[1] != G[1] or G[2] != ("load", _index(pf, wg)) or \
            U[2] != ("load", _index(pf, wu)) or D[2] != ("load", _index(pf, wd)):
        _fail(fam, "the program does not store down(up * silu(gate)) of x's gate and up "
                   "projections")
    bh, bi = _shape(a[i])[1], _shape(_buf(gate.args[1]))[0]
    if bh != Hd or bi != I:
        _fail(fam, f"blocks of {bh} hidden / {bi} intermediate columns: each workgroup reduces "
                   f"over one block and overwrites its output block, which is the MLP only for "
                   f"whole blocks (Block_h = {Hd}, Block_i = {I})")
    return Plan(fam, pf.params, [_index(pf, out)], dict(
        x=_index(pf, x), wg=_index(pf, wg), wu=_index(pf, wu), wd=_index(pf, wd),
        out=_index(pf, out), M=M, hidden=Hd, inter=I, dtype=dt, operand_dtype=operand))


def _seq_dim(pf, Q: Buffer) -> Optional[int]:
    """The dimension of ``Q`` that a tile copy slices by query block (``Q[bz, bx * block_M:..,
    by, :]`` in sequence-major programs, ``Q[bz, by, bx * block_M:.., :]`` in head-major ones)."""
    for op in _ops(pf, _COPY):
        src = op.args[0]
        if isinstance(src, BufferAccess) and src.buffer is Q:
            dims = [d for d, ix in enumerate(src.indices[:-1])
                    if isinstance(ix, slice) and ix.start is not None]
            if len(dims) == 1:
                return dims[0]
    return None


def _index_param(pf, tile: Buffer, src: Buffer) -> Optional[Buffer]:
    """The int32 parameter read inside the row index of the element stores that fill ``tile``
    from ``src`` (the cu_seqlens array of ``Q_unpad[q_start_idx + ..]``)."""
    for op in _ops(pf, ("store",)):
        v = op.args[2]
        if op.args[0] is not tile or not isinstance(v, BufferAccess) or v.buffer is not src:
            continue
        for ix in v.indices:
            if not isinstance(ix, Expr):
                continue
            for e in ix.walk():
                if isinstance(e, BufferAccess) and e.buffer.scope == "global" and \
                        e.buffer.dtype == "int32" and len(e.buffer.shape) == 1:
                    return e.buffer
    return None


def _flashattn_varlen(pf, qk, pv, Q, K, V, O) -> Plan:
    """examples/flash_attention/example_mha_fwd_varlen.py:222-358: unpadded Q/K/V/Output
    [tokens, heads, dim], int32 cu_seqlens_q / cu_seqlens_k [B + 1], scalar max_seqlen_q."""
    fam = "flashattn"
    shp, kshp = _shape(Q), _shape(K)
    if shp != _shape(O) or kshp != _shape(V) or len(kshp) != 3:
        _fail(fam, "variable-length Q, Output must be [tokens, heads, dim] and K, V "
                   "[tokens, kv_heads, dim]")
    UQ, H, D = shp
    UKV, Hkv, Dk = kshp
    if Dk != D or Hkv == 0 or H % Hkv:
        _fail(fam, f"K/V {kshp} do not group Q {shp} (same dim; heads a multiple of kv_heads)")
    tile_dts = {_buf(qk.args[0]).dtype, _buf(qk.args[1]).dtype, _buf(pv.args[0]).dtype,
                _buf(pv.args[1]).dtype}
    if not (Q.dtype == K.dtype == V.dtype == O.dtype) or tile_dts != {Q.dtype} or \
            Q.dtype not in ("bfloat16", "float16"):
        _fail(fam, "variable-length attention needs bfloat16 or float16 Q, K, V, Output and "
                   "tiles of the same dtype")
    cu_q = _index_param(pf, _buf(qk.args[0]), Q)
    cu_k = _index_param(pf, _buf(qk.args[1]), K)
    if cu_q is None or cu_k is None or cu_q is cu_k or _shape(cu_q) != _shape(cu_k):
        _fail(fam, "could not find the cu_seqlens_q / cu_seqlens_k parameters")
    B = _shape(cu_q)[0] - 1
    scalars = [p for p in pf.params if isinstance(p, ir.ScalarParam)]
    grid = pf.kernels[0].extents if pf.kernels else ()
    max_q = None
    for p in scalars:
        if any(isinstance(e, Expr) and p.name in e.free_vars() for e in grid):
            max_q = p
    if max_q is None:
        _fail(fam, "no scalar max_seqlen_q parameter sizes the grid")
    # The example's causal variant (:297-302) pre-fills -inf only where a query is on or below
    # the key's diagonal AND out of range, so in-range keys above the diagonal stay visible: it is
    # not causal attention, and no kernel here reproduces it.
    k_vars = {v.name for op in pf.ops if op.name == "loop_begin" and op.args[0].kind ==
              "pipelined" for v in op.args[0].vars}
    for op in pf.ops:
        if op.name == "branch" and isinstance(op.args[0], Expr):
            fv = op.args[0].free_vars()
            if any(n.startswith("bx") for n in fv) and fv & k_vars:
                _fail(fam, "the variable-length program's causal mask compares query and key "
                           "positions only together with the sequence bounds "
                           "(example_mha_fwd_varlen.py:298-302); only its non-causal form maps to "
                           "a kernel")
    acc_s = _buf(qk.args[2])
    sm_scale = None
    for op in _ops(pf, ("store",)):
        if op.args[0] is acc_s and isinstance(op.args[2], Expr) and op.args[2].has_op("exp2"):
            cs = [c for c in op.args[2].consts() if isinstance(c, float) and c > 0]
            if cs:
                sm_scale = cs[0] / LOG2E_REF
    if sm_scale is None:
        _fail(fam, "could not read the softmax scale")
    return Plan(fam, pf.params, [_index(pf, O)], dict(
        q=_index(pf, Q), k=_index(pf, K), v=_index(pf, V), o=_index(pf, O),
        cu_q=_index(pf, cu_q), cu_k=_index(pf, cu_k), max_q=_index(pf, max_q), varlen=True,
        B=B, total_q=UQ, total_k=UKV, H=H, H_kv=Hkv, D=D, causal=False, sm_scale=sm_scale,
        dtype=Q.dtype, operand_dtype=None))


def _page_size_from_trace(pf, bt: Buffer) -> Optional[int]:
    for op in pf.ops:
        for a in op.args:
            exprs = []
            if isinstance(a, BufferAccess):
                exprs = [ix.start for ix in a.indices if isinstance(ix, slice)]
                exprs += [ix for ix in a.indices if isinstance(ix, Expr)]
            for e in exprs:
                if not isinstance(e, Expr):
                    continue
                for n in e.walk():
                    if n.op == "mul" and isinstance(n.args[0], BufferAccess) and \
                            n.args[0].buffer is bt and n.args[1].op == "const":
                        return int(n.args[1].args[0])
    return None


def _mla(pf, names) -> Plan:
    """Paged (int32 BLOCK_TABLE [b, pages] + CACHE_SEQLENS [b]; example_mla_decode_paged.py) or
    non-paged (KV [b, seqlen_kv, 1, dv]; example_mla_decode.py and the TPU program
    tpu_demo/ppl/deepseek_mla/mla_decode.py, whose Q / Output carry a singleton query axis)
    MLA decode."""
    fam = "mla"
    ints = [p for p in pf.params if p.dtype == "int32"]
    bt = [p for p in ints if len(p.shape) == 2]
    sl = [p for p in ints if len(p.shape) == 1]
    paged = bool(ints)
    if paged and (len(bt) != 1 or len(sl) != 1 or len(ints) != 2):
        _fail(fam, "expected int32 BLOCK_TABLE [b, pages] and CACHE_SEQLENS [b]")
    bt = bt[0] if paged else None
    sl = sl[0] if paged else None
    g = [op for op in _ops(pf, _GEMM)]
    qk = [op for op in g if op.kwargs.get("transpose_B")]
    pv = [op for op in g if not op.kwargs.get("transpose_B")]
    kernels = {op.kernel for op in g}
    if len(qk) != 2 or len(pv) != 1 or len(kernels) != 1:
        _fail(fam, "expected Q@KV^T + Q_pe@K_pe^T and P@KV in one kernel")
    Q = _source_param(pf, _buf(qk[0].args[0]))
    KV = _source_param(pf, _buf(qk[0].args[1]))
    Qpe = _source_param(pf, _buf(qk[1].args[0]))
    Kpe = _source_param(pf, _buf(qk[1].args[1]))
    V = _source_param(pf, _buf(pv[0].args[1]))
    if None in (Q, KV, Qpe, Kpe) or V is not KV:
        _fail(fam, "could not trace Q, Q_pe, KV, K_pe (V must be the latent KV)")
    qshape = _shape(Q)
    if len(qshape) == 4 and qshape[2] == 1:  # TPU layout [b, hq, 1, d]
        b, hq, dv = qshape[0], qshape[1], qshape[3]
    elif len(qshape) == 3:
        b, hq, dv = qshape
    else:
        _fail(fam, f"Q must be [batch, heads, dim] or [batch, heads, 1, dim], got {qshape}")
    dpe = _shape(Qpe)[-1]
    O = glse = opart = None
    written = _written_params(pf)
    for p in written:
        s = _shape(p)
        if s == qshape:
            O = p
        elif len(s) == 3:
            glse = p
        elif len(s) == 4:
            opart = p
    if O is None:
        _fail(fam, "no Output parameter of Q's shape")
    for p in pf.params:  # glse / Output_partial may only be read (no-split form)
        s = _shape(p)
        if p in (Q, Qpe, KV, Kpe, bt, sl, O):
            continue
        if len(s) == 3 and glse is None and s[:2] == (b, hq):
            glse = p
        elif len(s) == 4 and opart is None and s[:2] == (b, hq) and s != qshape:
            opart = p
    kv_shape = _shape(KV)
    if paged:
        if len(kv_shape) != 3 or kv_shape[1] != 1 or kv_shape[2] != dv or \
                _shape(Kpe)[-1] != dpe:
            _fail(fam, "KV must be [rows, 1, dv] and K_pe [rows, 1, dpe] (one latent KV head)")
        if _shape(Qpe)[:2] != (b, hq) or _shape(sl) != (b,) or _shape(bt)[0] != b:
            _fail(fam, "batch/head dims disagree")
        max_pages = _shape(bt)[1]
        page = _page_size_from_trace(pf, bt)
        if page is None:
            page = kv_shape[0] // b // max_pages
        seqlen_kv = None
    else:
        if len(kv_shape) != 4 or kv_shape[0] != b or kv_shape[2] != 1 or kv_shape[3] != dv or \
                _shape(Kpe) != (b, kv_shape[1], 1, dpe) or _shape(Qpe)[:2] != (b, hq):
            _fail(fam, "non-paged KV must be [batch, seqlen_kv, 1, dv] and K_pe "
                       "[batch, seqlen_kv, 1, dpe] (one latent KV head)")
        seqlen_kv = kv_shape[1]
        page, max_pages = seqlen_kv, 1
    num_split = _shape(glse)[-1] if glse is not None else 1
    # the split form writes its partials: glse / Output_partial over the program's partition in
    # blocks of block_N tokens (the KV tile of the score gemm)
    partials = glse is not None and opart is not None and num_split > 1 and \
        any(p is glse for p in written) and any(p is opart for p in written)
    part_block = int(_shape(_buf(qk[0].args[1]))[0])
    if partials:
        if _shape(glse) != (b, hq, num_split) or _shape(opart) != (b, hq, num_split, dv):
            _fail(fam, f"glse {_shape(glse)} / Output_partial {_shape(opart)} are not "
                       f"[batch, heads, {num_split}] / [batch, heads, {num_split}, dv]")
        if glse.dtype != opart.dtype or glse.dtype not in ("float16", "bfloat16", "float32"):
            _fail(fam, "glse and Output_partial must share a float16, bfloat16 or float32 dtype")
        if not paged and seqlen_kv % (num_split * part_block):
            _fail(fam, f"seqlen_kv {seqlen_kv} does not split into {num_split} ranges of whole "
                       f"{part_block}-token tiles (the program's splits would overlap)")
    # scale: exp2(acc_s * c - max * c) with c = sm_scale * log2(e) (upstream programs), or the
    # TPU program's ppl_mul_C(scores, scores, sm_scale) before its natural-exp ppl_exp2
    sm_scale = None
    for op in _ops(pf, ("store",)):
        v = op.args[2]
        if isinstance(v, Expr) and v.has_op("exp2") and len(op.args[0].shape) == 2:
            cs = [c for c in v.consts() if isinstance(c, float) and c > 0]
            if cs:
                sm_scale = cs[0] / LOG2E_REF
                break
    if sm_scale is None and "ppl_exp" in names:
        acc_s = _buf(qk[0].args[2])
        cands = [op for op in _ops(pf, ("ppl_mul_C",)) if _buf(op.args[0]) is acc_s]
        if cands:
            sm_scale = _const(cands[0].args[2])
    if sm_scale is None:
        _fail(fam, "could not read the softmax scale")
    kv_scale = None
    if KV.dtype == "float8_e4m3":
        sc = [p for p in pf.params if p.dtype == "float32" and math.prod(_shape(p)) == 1]
        if len(sc) != 1:
            _fail(fam, "fp8 KV needs one float32 [1] scale parameter")
        kv_scale = _index(pf, sc[0])
    elif KV.dtype not in ("float16", "bfloat16"):
        _fail(fam, f"KV dtype {KV.dtype}")
    if Q.dtype not in ("float16", "bfloat16") or Qpe.dtype != Q.dtype:
        _fail(fam, f"Q dtype {Q.dtype}")
    if O.dtype not in ("float16", "bfloat16"):
        _fail(fam, f"Output dtype {O.dtype}")
    return Plan(fam, pf.params, [_index(pf, O)], dict(
        q=_index(pf, Q), q_pe=_index(pf, Qpe), kv=_index(pf, KV), k_pe=_index(pf, Kpe),
        block_table=None if bt is None else _index(pf, bt),
        seqlens=None if sl is None else _index(pf, sl), o=_index(pf, O),
        glse=None if glse is None else _index(pf, glse),
        o_partial=None if opart is None else _index(pf, opart), kv_scale=kv_scale, B=b, Hq=hq,
        dv=dv, dpe=dpe, page=page, max_pages=max_pages, num_split=num_split, sm_scale=sm_scale,
        paged=paged, seqlen_kv=seqlen_kv, q_dtype=Q.dtype, kv_dtype=KV.dtype, o_dtype=O.dtype,
        partials=partials, part_block=part_block))


def _sigmoid(pf, names) -> Plan:
    fam = "sigmoid"
    op = next(_ops(pf, ("ppl_sigmoid",)))
    x = _source_param(pf, _buf(op.args[1]))
    y = _sink_param(pf, _buf(op.args[0]))
    if x is None or y is None or _shape(x) != _shape(y):
        _fail(fam, "expected one input and one output of the same shape")
    if x.dtype != y.dtype or x.dtype not in ("float32", "float16", "bfloat16"):
        _fail(fam, f"dtypes {x.dtype} -> {y.dtype} (float32, float16 or bfloat16, matching)")
    if _symbolic(pf) != [(_index(pf, y), ("sigmoid", ("load", _index(pf, x))))]:
        _fail(fam, "the program stores something other than sigmoid(x)")
    return Plan(fam, pf.params, [_index(pf, y)], dict(
        x=_index(pf, x), y=_index(pf, y), n=math.prod(_shape(x)), dtype=x.dtype))


def _gather(pf, names) -> Plan:
    fam = "gather"
    op = next(_ops(pf, ("ppl_gather",)))
    out, param, index = (_buf(a) for a in op.args[:3])
    if None in (out, param, index) or any(b.scope != "global" for b in (out, param, index)):
        _fail(fam, "expected ppl_gather on global Output, Param and Index tensors")
    param_h = int(_const(op.args[3]))
    ps, os_, is_ = _shape(param), _shape(out), _shape(index)
    if len(ps) != 2 or len(os_) != 2 or os_[1] != ps[1] or math.prod(is_) != os_[0]:
        _fail(fam, f"shapes Param{ps} Index{is_} Output{os_} do not match a row gather")
    if param_h != ps[0]:
        _fail(fam, f"param_h {param_h} is not Param's row count {ps[0]}")
    if index.dtype not in ("uint32", "int32") or out.dtype != param.dtype:
        _fail(fam, "Index must be uint32 / int32 and Output share Param's dtype")
    return Plan(fam, pf.params, [_index(pf, out)], dict(
        param=_index(pf, param), index=_index(pf, index), out=_index(pf, out), rows=ps[0],
        hidden=ps[1], n=os_[0], dtype=param.dtype))


def _topk(pf, names) -> Plan:
    fam = "topk"
    op = next(_ops(pf, ("ppl_topk",)))
    vals, idx, src = (_buf(a) for a in op.args[:3])
    k, desc, length = (int(_const(a)) for a in op.args[3:6])
    if None in (vals, idx, src):
        _fail(fam, "expected ppl_topk on global tensors")
    if math.prod(_shape(src)) != length or math.prod(_shape(vals)) != length or \
            math.prod(_shape(idx)) != length:
        _fail(fam, f"length {length} does not match the tensors")
    if src.dtype not in ("float32", "int32", "uint32") or vals.dtype != src.dtype or \
            idx.dtype != "int32":
        _fail(fam, "src / values float32, int32 or uint32 and indices int32")
    if not 0 <= k <= length:
        _fail(fam, f"K = {k} outside [0, {length}]")
    return Plan(fam, pf.params, [_index(pf, vals), _index(pf, idx)], dict(
        src=_index(pf, src), values=_index(pf, vals), indices=_index(pf, idx), k=k,
        descending=bool(desc), length=length, dtype=src.dtype))


def _row_reduce(pf, names) -> Plan:
    fam = "row_reduce"
    reds = list(_ops(pf, ("ppl_reduce_max", "ppl_reduce_sum", "reduce_max", "reduce_sum")))
    if len(reds) != 1 or reds[0].kwargs.get("dim", 1) not in (1, -1):
        _fail(fam, "expected one row reduction over the last dim")
    op = reds[0]
    x = _source_param(pf, _buf(op.args[0]))
    y = _sink_param(pf, _buf(op.args[1]))
    if x is None or y is None:
        _fail(fam, "could not trace X and Y through the tile copies")
    xs, ys = _shape(x), _shape(y)
    if math.prod(ys) != math.prod(xs[:-1]):
        _fail(fam, f"Y{ys} does not hold one value per row of X{xs}")
    # one reduction of whole rows, stored as computed: a tile narrower than the row (or a
    # reduction repeated over column tiles) reduces only part of each row, and a max that does
    # not clear its output also takes the output's previous contents
    if op.loops or ("max" in op.name and not op.kwargs.get("clear", True)):
        _fail(fam, "expected one clearing reduction outside loops")
    want = ("rsum" if "sum" in op.name else "rmax", ("load", _index(pf, x)))
    if _symbolic(pf) != [(_index(pf, y), want)]:
        _fail(fam, "the program stores something other than the row reduction of X")
    maps = []
    for cop in _ops(pf, _COPY):
        src, dst = cop.args[0], cop.args[1]
        sb, db = _buf(src), _buf(dst)
        if sb is x:
            if not _covers_rows(cop, src, db, xs[-1]):
                _fail(fam, "the tile copy of X does not span whole rows")
            maps.append(_tile_map(pf, src, db, skip=-1))
        elif db is y:
            maps.append(_tile_map(pf, dst, sb, skip=-1))
    if len(maps) != 2 or maps[0] is None or maps[0][:-1] != maps[1][:len(maps[0]) - 1]:
        _fail(fam, "the tile copies of X and Y are not at one row-tile position")
    if x.dtype not in ("float32", "float16", "bfloat16") or \
            y.dtype not in ("float32", "float16", "bfloat16"):
        _fail(fam, f"dtypes {x.dtype} -> {y.dtype}")
    return Plan(fam, pf.params, [_index(pf, y)], dict(
        x=_index(pf, x), y=_index(pf, y), op="max" if "max" in op.name else "sum",
        rows=math.prod(xs[:-1]), cols=xs[-1], in_dtype=x.dtype, out_dtype=y.dtype))


# ------------------------------------------------------------------------------------------------
# elementwise tile programs: symbolic evaluation of the tile ops into a register program


_EW_BINARY = {"ppl_add": "add", "ppl_sub": "sub", "ppl_mul": "mul", "ppl_div": "div"}
_EW_CONSTOP = {"ppl_add_C": "add", "ppl_mul_C": "mul"}
_EW_OPCODE = {"load": 0, "const": 1, "add": 2, "sub": 3, "mul": 4, "div": 5, "exp": 6, "rsqrt": 7,
              "sigmoid": 8, "round": 9, "store": 10}
_EW_DTYPE = {"float32": 2, "float16": 0, "bfloat16": 1}  # enum tlm_dtype
_EW_BCAST = {"full": 0, "row": 1, "col": 2, "scalar": 3}


def _grid_var_extent(pf, e) -> Optional[int]:
    """Extent of the kernel grid dimension whose variable is ``e`` (None if it is not one)."""
    if not isinstance(e, Expr) or e.op != "var" or not pf.kernels:
        return None
    # the kernel that binds this variable object (a program may launch several kernels, each
    # with its own bx, by), else a variable of the same name in the first kernel
    pairs = [(v, ext) for k in pf.kernels for v, ext in zip(k.vars, k.extents) if v is e]
    if not pairs:
        k = pf.kernels[0]
        pairs = [(v, ext) for v, ext in zip(k.vars, k.extents)
                 if isinstance(v, Expr) and v.args[0] == e.args[0]]
    if not pairs:
        return None
    try:
        return int(ir.const_value(pairs[0][1]))
    except (TypeError, ValueError):
        return None


def _eval_int(e, v):
    """Integer value of an index expression of +, -, * with every variable set to ``v``."""
    if isinstance(e, bool):
        return None
    if isinstance(e, int):
        return e
    if isinstance(e, Expr):
        if e.op == "const" and isinstance(e.args[0], int):
            return e.args[0]
        if e.op == "var":
            return v
        if e.op in ("add", "sub", "mul") and len(e.args) == 2:
            a, b = _eval_int(e.args[0], v), _eval_int(e.args[1], v)
            if a is None or b is None:
                return None
            return a + b if e.op == "add" else a - b if e.op == "sub" else a * b
    return None


def _extent_value(ex) -> Optional[int]:
    """A region extent as an integer: a constant, or a slice length such as
    ``(bx + 1) * 32 - bx * 32`` that takes one value whatever the grid variables (checked at
    three settings of them); None otherwise."""
    try:
        return int(ir.const_value(ex))
    except (TypeError, ValueError):
        pass
    vals = {_eval_int(ex, v) for v in (0, 1, 7)}
    return vals.pop() if len(vals) == 1 and None not in vals else None


def _eval_env(e, env: Dict[str, int]):
    """Integer value of an index expression of +, -, * with variables from ``env`` (others 0)."""
    if isinstance(e, bool):
        return None
    if isinstance(e, int):
        return e
    if isinstance(e, Expr):
        if e.op == "const" and isinstance(e.args[0], int):
            return e.args[0]
        if e.op == "var":
            return env.get(e.args[0], 0)
        if e.op in _INT_OPS and len(e.args) == 2:
            a, b = _eval_env(e.args[0], env), _eval_env(e.args[1], env)
            if a is None or b is None or (e.op in ("mod", "floordiv") and b == 0):
                return None
            return int(_INT_OPS[e.op](a, b))
    return None


_INT_OPS = {"add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
            "mod": lambda a, b: a % b, "floordiv": lambda a, b: a // b,
            "eq": lambda a, b: a == b, "ne": lambda a, b: a != b, "lt": lambda a, b: a < b,
            "le": lambda a, b: a <= b, "gt": lambda a, b: a > b, "ge": lambda a, b: a >= b,
            "and": lambda a, b: bool(a) and bool(b), "or": lambda a, b: bool(a) or bool(b)}


def _covers_rows(op, access, tile: Buffer, ncols: int, d: int = -1) -> bool:
    """Whether the tile copy ``access`` of ``op`` reads or writes whole rows of its parameter
    over all iterations of the loops around it: column starts 0, w, 2w, ... (in any order, each
    once) for a tile w columns wide, together spanning the ``ncols`` columns. ``d`` names
    another dimension to check the same way (the k dimension of a GEMM operand)."""
    if isinstance(access, Buffer):
        return True
    starts, exts = access.region(tile.shape)
    w = _extent_value(exts[d])
    if w is None or w <= 0:
        return False
    names, ranges = [], []
    for lp in op.loops or ():
        for v, ext in zip(lp.vars, lp.extents):
            n = _extent_value(ext)
            if n is None or n <= 0 or not isinstance(v, Expr):
                return False
            names.append(v.args[0])
            ranges.append(n)
    if math.prod(ranges) > 4096:
        return False
    cols = []
    for it in range(math.prod(ranges)):
        env, r = {}, it
        for name, n in zip(names, ranges):
            env[name], r = r % n, r // n
        c = _eval_env(starts[d], env)
        if c is None:
            return False
        cols.append(c)
    e = len(cols)
    return sorted(cols) == [i * w for i in range(e)] and (e - 1) * w < ncols <= e * w


def _tile_map(pf, access, tile: Buffer, skip: Optional[int] = None):
    """Grid mapping of the tile copy ``access`` of a global parameter, or None when the copy is
    not the (i, j)-th tile of a grid that covers the parameter exactly. Per dimension the entry
    is None (the whole or unit dimension, or a tile as long as the dimension) or (grid variable
    name, tile extent) for a start of grid_var * t with extent t and a grid extent of
    ceil(dim / t). ``skip``: a dimension that is not examined (entry None), such as the
    column dimension of a copy stepped over columns by a loop."""
    buf = access.buffer if isinstance(access, BufferAccess) else access
    dims = _shape(buf)
    if isinstance(access, Buffer):
        return [None] * len(dims)
    starts, exts = access.region(tile.shape)
    out = []
    for d, (st, ex) in enumerate(zip(starts, exts)):
        if skip is not None and d == skip % len(dims):
            out.append(None)
            continue
        t = _extent_value(ex)
        try:
            s0 = int(ir.const_value(st))
        except (TypeError, ValueError):
            s0 = None
        if s0 == 0 and (t == dims[d] or dims[d] == 1):
            out.append(None)
            continue
        if isinstance(st, Expr) and st.op == "var":  # a grid variable alone: unit tiles
            var, c = st, 1
        elif isinstance(st, Expr) and st.op == "mul":
            a, b = st.args
            var, c = (a, b) if isinstance(b, Expr) and b.op == "const" else (b, a)
            if not (isinstance(c, Expr) and c.op == "const"):
                return None
            c = int(c.args[0])
        else:
            return None
        if t is None:
            tdims = list(tile.shape)
            t = int(ir.const_value(tdims[d - (len(dims) - len(tdims))])) if len(tdims) else 1
        if t != c or _grid_var_extent(pf, var) != -(-dims[d] // c):
            return None
        out.append(None if t >= dims[d] else (var.args[0], t))
    return out


def _tiles_cover(pf, access, tile: Buffer) -> bool:
    """Whether the tile copy ``access`` takes one tile of a grid covering its parameter."""
    return _tile_map(pf, access, tile) is not None


def _elementwise(pf, names) -> Plan:
    fam = "elementwise"
    if len(pf.kernels) != 1:
        _fail(fam, "expected one kernel")
    writes = _written_params(pf)
    if not writes:
        _fail(fam, "no output parameter")
    full = _shape(writes[0])
    if any(_shape(w) != full for w in writes):
        _fail(fam, "outputs of different shapes")
    rows = math.prod(full[:-1]) if len(full) > 1 else 1
    cols = full[-1]
    nodes: List[tuple] = []  # (kind, a, b, imm)
    memo: Dict[tuple, int] = {}

    def node(kind, a=-1, b=-1, imm=0):
        key = (kind, a, b, imm)
        if key not in memo:
            memo[key] = len(nodes)
            nodes.append(key)
        return memo[key]

    def rounded(n, dtype):
        return n if dtype == "float32" else node("round", n, imm=_EW_DTYPE[dtype])

    inputs: List[Buffer] = []
    kinds: List[str] = []
    consts: List[float] = []
    value: Dict[int, int] = {}  # id(tile) -> node
    stores: List[tuple] = []    # (output parameter, node)

    stored: List[Buffer] = []
    maps: List[tuple] = []      # (kind, grid map) of every global tile copy

    def load(p):
        if any(p is q for q in stored):
            # a later copy from a parameter the program has written would read the stored
            # values; the register program reads each input once, before any store
            _fail(fam, f"parameter {p!r} is copied from after the program stores to it")
        s = _shape(p)
        n = math.prod(s)
        if s == full:
            kind = "full"
        elif n == 1:
            kind = "scalar"
        elif n == rows and s[-1] == 1:
            kind = "row"
        elif n == cols and len(s) >= 1 and s[-1] == cols:
            kind = "col"
        else:
            _fail(fam, f"parameter {p!r} does not broadcast onto the {full} output")
        for k, q in enumerate(inputs):
            if q is p:
                return node("load", imm=k)
        inputs.append(p)
        kinds.append(kind)
        return node("load", imm=len(inputs) - 1)

    def const(v, dtype):
        v = float(v)
        if v not in consts:
            consts.append(v)
        return rounded(node("const", imm=consts.index(v)), dtype)

    def get(b):
        b = _buf(b)
        if b is None or id(b) not in value:
            _fail(fam, f"tile {b!r} is read before it is written")
        return value[id(b)]

    for op in _ops(pf):
        n = op.name
        if n in _COPY:
            src, dst = op.args[0], op.args[1]
            sb, db = _buf(src), _buf(dst)
            if sb is None or db is None:
                _fail(fam, "copy operands must be buffers")
            if sb.scope == "global" and db.scope != "global":
                m = _tile_map(pf, src, db)
                if m is None:
                    _fail(fam, f"the copy from {sb!r} is not one tile of a grid covering it")
                value[id(db)] = rounded(load(sb), db.dtype)
                maps.append((kinds[[q is sb for q in inputs].index(True)], m, sb))
            elif sb.scope != "global" and db.scope == "global":
                m = _tile_map(pf, dst, sb)
                if m is None:
                    _fail(fam, f"the copy to {db!r} is not one tile of a grid covering it")
                stores.append((db, get(sb)))
                stored.append(db)
                maps.append(("out", m, db))
            elif sb.scope != "global" and db.scope != "global":
                value[id(db)] = rounded(get(sb), db.dtype)
            else:
                _fail(fam, "global-to-global copies are not tile programs")
        elif n in _FILL_OPS:
            b = _buf(op.args[0])
            value[id(b)] = const(_const(op.args[1]), b.dtype)
        elif n in _EW_BINARY:
            out, x, y = (_buf(a) for a in op.args[:3])
            value[id(out)] = rounded(node(_EW_BINARY[n], get(x), get(y)), out.dtype)
        elif n in _EW_CONSTOP:
            out, x = _buf(op.args[0]), _buf(op.args[1])
            c = const(_const(op.args[2]), x.dtype)
            value[id(out)] = rounded(node(_EW_CONSTOP[n], get(x), c), out.dtype)
        elif n == "ppl_exp":
            out = _buf(op.args[0])
            value[id(out)] = rounded(node("exp", get(out)), out.dtype)
        elif n in ("ppl_rsqrt", "ppl_sigmoid"):
            out, x = _buf(op.args[0]), _buf(op.args[1])
            value[id(out)] = rounded(node(n[4:], get(x)), out.dtype)
        else:
            _fail(fam, f"op {n} is not an elementwise tile op")
    if not stores:
        _fail(fam, "nothing is stored")
    # every tile copy must address the same element grid: the kernel applies the program to
    # element (r, c) of every operand, so an input tile taken at another grid position than
    # the output tile (a tile transpose, a shifted tile) has no elementwise meaning here
    out_map = next(m for k, m, _ in maps if k == "out")
    for kind, m, p in maps:
        if kind == "scalar":
            continue
        if kind in ("out", "full"):
            ok = m == out_map
        elif kind == "row":
            ok = len(m) == len(out_map) and m[:-1] == out_map[:-1] and m[-1] is None
        else:  # col
            ok = m[-1] == out_map[-1]
        if not ok:
            _fail(fam, f"the tile copy of {p!r} is not at the output tile's grid position")
    outs: List[Buffer] = []
    for p, _ in stores:
        if all(p is not q for q in outs):
            outs.append(p)
    if len(inputs) > 8 or len(outs) > 4 or len(consts) > 16:
        _fail(fam, "more than 8 inputs, 4 outputs or 16 constants")
    # register allocation over the nodes the stores need, in program (topological) order
    need = set()

    def mark(i):
        if i in need or i < 0:
            return
        need.add(i)
        mark(nodes[i][1])
        mark(nodes[i][2])

    for _, i in stores:
        mark(i)
    last_use: Dict[int, int] = {}
    order = sorted(need)
    for pos, i in enumerate(order):
        for a in nodes[i][1:3]:
            if a >= 0:
                last_use[a] = pos
    final = {i: len(order) + k for k, (_, i) in enumerate(stores)}
    for i, pos in final.items():
        last_use[i] = max(last_use.get(i, -1), pos)
    slot: Dict[int, int] = {}
    free = list(range(8))
    code: List[int] = []
    for pos, i in enumerate(order):
        kind, a, b, imm = nodes[i]
        sa, sb = slot.get(a, 0), slot.get(b, 0)
        for x in (a, b):  # operands whose last use is here free their slot for the result
            if x >= 0 and last_use.get(x) == pos and x in slot and slot[x] not in free:
                free.append(slot[x])
        if not free:
            _fail(fam, "the program needs more than 8 live values")
        d = min(free)
        free.remove(d)
        slot[i] = d
        code.append(_EW_OPCODE[kind] | d << 8 | sa << 12 | sb << 16 | imm << 20)
    for p, i in stores:
        code.append(_EW_OPCODE["store"] | slot[i] << 12 | outs.index(p) << 20)
    if len(code) > 64:
        _fail(fam, "more than 64 instructions")
    return Plan(fam, pf.params, [_index(pf, p) for p in outs], dict(
        inputs=[_index(pf, p) for p in inputs], bcast=[_EW_BCAST[k] for k in kinds],
        outputs=[_index(pf, p) for p in outs], code=code, consts=consts, rows=rows, cols=cols))


def recognize(pf) -> Plan:
    """Return the :class:`Plan` for ``pf`` or raise :class:`UnsupportedProgram`."""
    names = set(_op_names(pf))
    ints = [p for p in pf.params if p.dtype == "int32"]
    n_gemm = sum(1 for op in _ops(pf, _GEMM))
    try:
        if n_gemm == 3 and "ppl_div" in names and not names & {"ppl_reduce_max", "reduce_max"}:
            return _audit(pf, _mlp(pf, names))
        if n_gemm >= 3:
            return _audit(pf, _mla(pf, names))
        if n_gemm == 2 and names & {"ppl_reduce_max", "reduce_max"}:
            return _audit(pf, _flashattn(pf, names))
        if n_gemm == 1 and not names & {"ppl_exp", "ppl_reduce_max", "reduce_max"}:
            return _audit(pf, _gemm(pf, names))
        if "ppl_rope_add" in names:
            return _audit(pf, _rope(pf, names))
        if {"ppl_reduce_sum", "ppl_rsqrt"} <= names:
            return _audit(pf, _rmsnorm(pf, names))
        # tile programs of copies, fills and elementwise ops (a fill-only program, such as the
        # symbolic-shape fill of tpu_demo/ppl/matmul.py, stores a constant)
        ew = n_gemm == 0 and names <= set(_ALLOWED_OPS["elementwise"]) and \
            bool(names & (set(_ALLOWED_OPS["elementwise"]) - set(_COPY)))
        if {"ppl_exp", "ppl_div"} <= names or "ppl_sigmoid" in names:
            # the dedicated SwiGLU / sigmoid kernels, else the general elementwise program
            try:
                fam = _swiglu if "ppl_sigmoid" not in names else _sigmoid
                return _audit(pf, fam(pf, names))
            except UnsupportedProgram:
                if not ew:
                    raise
                return _audit(pf, _elementwise(pf, names))
        if "ppl_gather" in names:
            return _audit(pf, _gather(pf, names))
        if "ppl_topk" in names:
            return _audit(pf, _topk(pf, names))
        if n_gemm == 0 and len(names & {"ppl_reduce_max", "ppl_reduce_sum", "reduce_max",
                                        "reduce_sum"}) == 1 and \
                not names & {"ppl_exp", "ppl_rsqrt", "ppl_div", "ppl_mul"}:
            return _audit(pf, _row_reduce(pf, names))
        if ew:
            return _audit(pf, _elementwise(pf, names))
    except UnsupportedProgram:
        raise
    except (TypeError, ValueError, IndexError) as e:  # malformed trace
        raise UnsupportedProgram(f"{pf.name}: could not analyse program: {e}") from e
    raise UnsupportedProgram(
        f"{pf.name}: no gfx950 kernel matches this program (ops: {sorted(names)}). Supported "
        f"families: rmsnorm, gemm, rope, swiglu, flashattn, mla, mlp, sigmoid, gather, topk, "
        f"row_reduce, elementwise")
