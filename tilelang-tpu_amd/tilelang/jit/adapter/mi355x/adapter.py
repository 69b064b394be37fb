"""The mi355x kernel adapter: the callable that ``tilelang.compile`` returns.

Both call conventions of the reference are kept:
  * TPU convention (tilelang/jit/adapter/cython/adapter.py:218-246): the caller passes ALL
    parameters in prim_func order; outputs are written in place; the call returns ``0``.
    Tensors may live on the host (the demos pass CPU tensors): they are copied to the GPU and
    the outputs copied back, as the reference copies through host buffers.
  * GPU convention (tilelang/jit/adapter/cython/cython_wrapper.pyx:68-163): the caller passes
    the inputs only; outputs are allocated on the inputs' device and returned (one tensor, or a
    list for several outputs). Count, dtype, static shape and device mismatches raise ValueError.
The convention is chosen by the number of arguments.
"""
from typing import Any, List

import torch

from ....language import ir
from ..base import BaseKernelAdapter
from . import ops
from .recognize import recognize


_TORCH_DT = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


def _cast_to(v: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """A copy of ``v`` in dtype ``dt`` made by the library's cast kernel (round to nearest
    even)."""
    o = torch.empty(v.shape, dtype=dt, device=v.device)
    ops.cast(v, o)
    return o


def _eval_extent(s, env):
    """Integer value of a tensor extent under the symbolic binding ``env`` (None if unbound)."""
    if isinstance(s, int):
        return s
    if ir.sym_names(s) - set(env):
        return None
    v = ir.substitute(s, env)
    return int(ir.const_value(v))


def _stream_key(dev):
    """Workspaces are kept per device and stream: the kernels of one stream run in order, so a
    stream's calls can share its workspace, while calls on two streams may overlap."""
    return (dev, torch.cuda.current_stream(dev).cuda_stream)


def _run_plan(plan, t: List[torch.Tensor], workspace_cache: dict):
    a = plan.attrs
    f = plan.family
    odt = _TORCH_DT.get(a.get("operand_dtype"))  # fp32 programs with 16-bit matrix tiles
    if f == "rmsnorm":
        w = None if a["w"] is None else t[a["w"]]
        ops.rmsnorm(t[a["x"]], w, t[a["y"]], a["eps"])
    elif f == "swiglu":
        ops.swiglu(t[a["gate"]], t[a["up"]], t[a["out"]])
    elif f == "rope":
        k = None if a["k"] is None else t[a["k"]]
        ko = None if a["k_out"] is None else t[a["k_out"]]
        ops.rope(t[a["q"]], t[a["cos"]], t[a["sin"]], t[a["q_out"]], k, ko)
    elif f == "gemm":
        ops.gemm(t[a["a"]], t[a["b"]], t[a["c"]], a["trans_b"], operand_dtype=odt)
    elif f == "flashattn" and a.get("varlen"):
        ops.flash_attn_varlen_fwd(t[a["q"]], t[a["k"]], t[a["v"]], t[a["cu_q"]], t[a["cu_k"]],
                                  t[a["max_q"]], t[a["o"]], a["causal"], a["sm_scale"])
    elif f == "flashattn" and a.get("layout") == "bshd_kv":
        # split-KV inference program: partial outputs and log2 sum-exp per key split written to
        # the program's glse / Output_partial, then their combine into Output
        q = t[a["q"]]
        need = ops.flash_attn_splitkv_workspace_bytes(a["B"], a["S"], a["S_kv"], a["H"], a["D"],
                                                      a["num_split"])
        key = (_stream_key(q.device), "splitkv")
        ws = workspace_cache.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
            workspace_cache[key] = ws
        ops.flash_attn_splitkv_fwd(q, t[a["k"]], t[a["v"]], t[a["glse"]], t[a["partial"]],
                                   t[a["o"]], a["num_split"], a["sm_scale"], ws)
    elif f == "flashattn" and a.get("layout") == "bhsd":
        ops.flash_attn_bhsd_fwd(t[a["q"]], t[a["k"]], t[a["v"]], t[a["o"]], a["causal"],
                                a["sm_scale"])
    elif f == "flashattn":
        ops.flash_attn_fwd(t[a["q"]], t[a["k"]], t[a["v"]], t[a["o"]], a["causal"], a["sm_scale"],
                           operand_dtype=odt)
    elif f == "mlp":
        # gate / up projections into 16-bit temporaries, SiLU(gate) * up, down projection
        x, out = t[a["x"]], t[a["out"]]
        wg, wu, wd = t[a["wg"]], t[a["wu"]], t[a["wd"]]
        M, I = a["M"], a["inter"]
        if odt is not None:
            # all-fp32 program: its fp32 tiles are copied to 16-bit tiles for the gemms, whose
            # 16-bit result of the down projection is copied to the fp32 output
            x, wg, wu, wd = (_cast_to(v, odt) for v in (x, wg, wu, wd))
        gate = torch.empty(M, I, dtype=x.dtype, device=x.device)
        up = torch.empty_like(gate)
        ops.gemm(x, wg, gate, True)
        ops.gemm(x, wu, up, True)
        ops.swiglu(gate, up, gate)
        if odt is None:
            ops.gemm(gate, wd, out, True)
        else:
            d16 = torch.empty(out.shape, dtype=odt, device=out.device)
            ops.gemm(gate, wd, d16, True)
            ops.cast(d16, out)
    elif f == "sigmoid":
        ops.sigmoid(t[a["x"]], t[a["y"]])
    elif f == "gather":
        ops.gather_rows(t[a["param"]], t[a["index"]], t[a["out"]])
    elif f == "topk":
        ops.topk(t[a["src"]], a["k"], a["descending"], t[a["values"]], t[a["indices"]])
    elif f == "row_reduce":
        ops.row_reduce(t[a["x"]], t[a["y"]], a["op"])
    elif f == "mla":
        q = t[a["q"]]
        dev = q.device
        # A program that does not write its partials leaves the key split to the kernels: about
        # one workgroup per CU (B * splits workgroups), as the balanced FP8 decode and the split
        # kernel both launch. The split program writes one partial per split of its own
        # partition, so it runs with its num_split.
        ns = a["num_split"] if a.get("partials") else max(1, min(64, -(-256 // max(1, a["B"]))))
        need = ops.mla_workspace_bytes(a["B"], a["Hq"], a["dv"], ns)
        ws = workspace_cache.get(_stream_key(dev))
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
            workspace_cache[_stream_key(dev)] = ws
        kvs = None if a["kv_scale"] is None else t[a["kv_scale"]]
        B, Hq, dv, dpe = a["B"], a["Hq"], a["dv"], a["dpe"]
        if a["paged"]:
            bt, sl = t[a["block_table"]], t[a["seqlens"]]
            qq, qpe, o = q, t[a["q_pe"]], t[a["o"]]
        else:
            # non-paged cache [B, S, 1, d]: token t of sequence b is row b * S + t, i.e. one page
            # of S tokens per sequence under the identity table (kept per device, stream and shape)
            key = (_stream_key(dev), "identity", B, a["seqlen_kv"])
            if key not in workspace_cache:
                workspace_cache[key] = (
                    torch.arange(B, dtype=torch.int32, device=dev).view(B, 1),
                    torch.full((B,), a["seqlen_kv"], dtype=torch.int32, device=dev))
            bt, sl = workspace_cache[key]
            qq = q.view(B, Hq, dv)
            qpe = t[a["q_pe"]].view(B, Hq, dpe)
            o = t[a["o"]].view(B, Hq, dv)
        g = op = None
        if a.get("partials"):  # the split program writes glse / Output_partial
            g, op = t[a["glse"]], t[a["o_partial"]]
            if not a["paged"]:
                g = g.view(B, Hq, a["num_split"])
                op = op.view(B, Hq, a["num_split"], dv)
        ops.mla_decode(qq, qpe, t[a["kv"]], t[a["k_pe"]], bt, sl, o, ws, a["page"], ns,
                       a["sm_scale"], kvs, glse=g, o_partial=op,
                       part_block=a.get("part_block", 64))
    elif f == "elementwise":
        ops.elementwise([t[i] for i in a["inputs"]], a["bcast"], [t[i] for i in a["outputs"]],
                        a["code"], a["consts"], a["rows"], a["cols"])
    else:  # pragma: no cover - recognizer only emits the families above
        raise RuntimeError(f"no runner for family {f}")


class MI355XKernelAdapter(BaseKernelAdapter):

    def __init__(self, params, result_idx, plan, prim_func=None):
        self.plan = plan
        self.prim_func = prim_func
        # symbolic extents: the plan above is the compile-time trial; each call recognises the
        # program specialised to its argument shapes (cached per binding)
        self.dynamic = any(p.is_dynamic() for p in params)
        self._plans = {}
        self._ws = {}
        super().__init__(None, params, result_idx)
        # the recognizer knows which parameters the program writes
        if not self.result_idx:
            self.result_idx = list(plan.out_idx)

    def get_kernel_source(self, kernel_only: bool = False) -> str:
        return (f"// gfx950 kernel family {self.plan.describe()}\n"
                f"// dispatched through libtlmi355x.so (include/tlmi355x.h)\n")

    def _check(self, i, t, env=None):
        p = self.params[i]
        if p.is_scalar():  # a plain Python int, as cython_wrapper.pyx:117-122 passes it
            if isinstance(t, bool) or not isinstance(t, int):
                raise ValueError(f"parameter {i} is a scalar {p.dtype}: pass a Python int, got "
                                 f"{type(t)}")
            return
        if not isinstance(t, torch.Tensor):
            raise ValueError(f"parameter {i} must be a torch.Tensor, got {type(t)}")
        if t.dtype != p.dtype:
            raise ValueError(f"Buffer dtype mismatch for parameter {i}: expected {p.dtype}, "
                             f"got {t.dtype}")
        if not p.is_dynamic():
            if list(t.shape) != [int(s) for s in p.shape]:
                raise ValueError(f"Static shape mismatch for parameter {i}: expected "
                                 f"{list(p.shape)}, got {list(t.shape)}")
            return
        # symbolic extents (T.symbolic): a plain variable is bound by the first argument that
        # carries it; _check_bound then compares every extent with its value under the binding
        if t.dim() != len(p.shape):
            raise ValueError(f"Dimension mismatch for parameter {i}: expected {len(p.shape)} "
                             f"dims, got {t.dim()}")
        for s, n in zip(p.shape, t.shape):
            if isinstance(s, ir.Var) and s.name not in env:
                env[s.name] = int(n)

    def _check_bound(self, i, t, env):
        """Every extent of a symbolic-shape parameter equals its value under the binding that
        all arguments made (so an extent such as 2 * m is checked even when m is bound by a
        later argument)."""
        p = self.params[i]
        for d, (s, n) in enumerate(zip(p.shape, t.shape)):
            v = _eval_extent(s, env)
            if v is None:
                raise ValueError(f"extent {s!r} of parameter {i} dim {d} is not bound by any "
                                 f"input tensor")
            if v != int(n):
                raise ValueError(f"Shape mismatch for parameter {i} dim {d}: expected {s!r} = "
                                 f"{v} under {env}, got {int(n)}")

    def _plan_for(self, env):
        """The plan of the program specialised to the bound symbolic extents (cached)."""
        if not self.dynamic:
            return self.plan
        names = self.prim_func.symbolic_vars()
        missing = [n for n in names if n not in env]
        if missing:
            raise ValueError(f"symbolic extents {missing} are not bound by any input tensor")
        key = tuple(env[n] for n in names)
        plan = self._plans.get(key)
        if plan is None:
            plan = recognize(self.prim_func.specialize({n: env[n] for n in names}))
            self._plans[key] = plan
        return plan

    def _convert_torch_func(self):

        def forward(*args: Any):
            n = len(self.params)
            outs = self.result_idx
            if len(args) == n:
                inplace = True
                full = list(args)
            elif len(args) == n - len(outs):
                inplace = False
                it = iter(args)
                full = [None if i in outs else next(it) for i in range(n)]
            else:
                raise ValueError(f"Expected {n} arguments (all parameters, outputs written in "
                                 f"place) or {n - len(outs)} (inputs only), got {len(args)}")
            env: dict = {}
            for i, t in enumerate(full):
                if t is not None:
                    self._check(i, t, env)
            if self.dynamic:
                for i, t in enumerate(full):
                    if isinstance(t, torch.Tensor) and self.params[i].is_dynamic():
                        self._check_bound(i, t, env)
            plan = self._plan_for(env)
            ins = [t for t in full if isinstance(t, torch.Tensor)]
            if not torch.cuda.is_available():
                raise RuntimeError("no HIP device visible: the mi355x target runs on gfx950 only "
                                   "and has no CPU fallback")
            devs = {t.device for t in ins}
            if len(devs) > 1:
                raise ValueError(f"Buffer device mismatch: arguments on {sorted(map(str, devs))}")
            home = next(iter(devs)) if devs else torch.device("cuda", torch.cuda.current_device())
            gpu = home if home.type == "cuda" else torch.device(
                "cuda", torch.cuda.current_device())
            dev_t = []
            for i, t in enumerate(full):
                if t is None:
                    p = self.params[i]
                    shape = [_eval_extent(s, env) for s in p.shape]
                    if any(v is None for v in shape):
                        raise ValueError(f"the shape {list(p.shape)} of output {i} is not bound "
                                         f"by the inputs")
                    dev_t.append(torch.empty(shape, dtype=p.dtype, device=gpu))
                elif not isinstance(t, torch.Tensor):  # scalar argument
                    dev_t.append(t)
                elif t.device != gpu:
                    dev_t.append(t.to(gpu))
                else:
                    dev_t.append(t)
            _run_plan(plan, dev_t, self._ws)
            if inplace:
                for i in outs:
                    if full[i].data_ptr() != dev_t[i].data_ptr():
                        full[i].copy_(dev_t[i])
                return 0
            res = [dev_t[i] if home.type == "cuda" else dev_t[i].to(home) for i in outs]
            return res[0] if len(res) == 1 else res

        return forward
