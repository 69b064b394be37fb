"""Torch-tensor front of each C-ABI entry point.

These functions take device tensors that the caller allocated (torch is only the allocator and
the stream provider), check dtype/shape/contiguity, and call libtlmi355x.so on the current
stream. They are what the mi355x kernel adapter dispatches to, and can be called directly.
"""
from typing import Optional

import torch

from . import lib

_DT = {torch.float16: lib.F16, torch.bfloat16: lib.BF16, torch.float32: lib.F32,
       torch.float8_e4m3fn: lib.F8E4M3, torch.float8_e5m2: lib.F8E5M2, torch.int32: lib.I32,
       torch.uint32: lib.U32}
_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


def dtype_code(dt: torch.dtype) -> int:
    if dt not in _DT:
        raise ValueError(f"dtype {dt} is not supported by the mi355x kernels")
    return _DT[dt]


def _dev(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t)}")
        if t.device.type != "cuda":
            raise ValueError(f"tensor on {t.device}: the mi355x kernels take HIP device tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    lib.ensure_device(dev.index if dev.index is not None else torch.cuda.current_device())
    return dev


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _contig(name, t):
    if t is not None and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def rmsnorm(x: torch.Tensor, w: Optional[torch.Tensor], y: torch.Tensor, eps: float):
    """y = cast(x * rsqrt(mean(x^2) + eps) * w) over the last dim."""
    dev = _dev(x, w, y)
    for n, t in (("x", x), ("w", w), ("y", y)):
        _contig(n, t)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError("y must match x in shape and dtype")
    if w is not None and (w.numel() != cols or w.dtype != x.dtype):
        raise ValueError(f"w must have {cols} elements of dtype {x.dtype}")
    lib.call("tlm_rmsnorm", _ptr(x), _ptr(w), _ptr(y), rows, cols, float(eps),
             dtype_code(x.dtype), _stream(dev))
    return y


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor):
    """out = up * silu(gate), fp32 math."""
    dev = _dev(gate, up, out)
    for n, t in (("gate", gate), ("up", up), ("out", out)):
        _contig(n, t)
    if not (gate.shape == up.shape == out.shape) or not (gate.dtype == up.dtype == out.dtype):
        raise ValueError("gate, up and out must share shape and dtype")
    lib.call("tlm_swiglu", _ptr(gate), _ptr(up), _ptr(out), gate.numel(), dtype_code(gate.dtype),
             _stream(dev))
    return out


def rope(q: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, q_out: torch.Tensor,
         k: Optional[torch.Tensor] = None, k_out: Optional[torch.Tensor] = None):
    """Interleaved RoPE. q/k are [tokens, heads, dim] (or [tokens, dim]); cos/sin [tokens, dim]."""
    dev = _dev(q, cos, sin, q_out, k, k_out)
    for n, t in (("q", q), ("cos", cos), ("sin", sin), ("q_out", q_out), ("k", k),
                 ("k_out", k_out)):
        _contig(n, t)
    dim = q.shape[-1]
    tokens = cos.numel() // dim if dim else 0
    if cos.shape != sin.shape or cos.shape[-1] != dim:
        raise ValueError("cos and sin must be [tokens, dim]")
    hq = q.numel() // (tokens * dim) if tokens else 1
    if hq * tokens * dim != q.numel() or q_out.shape != q.shape:
        raise ValueError(f"q {tuple(q.shape)} does not split into {tokens} tokens x heads x {dim}")
    hk = 0
    if k is not None:
        hk = k.numel() // (tokens * dim) if tokens else 1
        if hk * tokens * dim != k.numel() or k_out is None or k_out.shape != k.shape:
            raise ValueError("k/k_out do not match the token count of the tables")
    dts = {t.dtype for t in (q, cos, sin, q_out, k, k_out) if t is not None}
    if len(dts) != 1:
        raise ValueError(f"all RoPE tensors must share one dtype, got {dts}")
    lib.call("tlm_rope", _ptr(q), _ptr(k), _ptr(cos), _ptr(sin), _ptr(q_out), _ptr(k_out), tokens,
             hq, hk, dim, dtype_code(q.dtype), _stream(dev))
    return q_out


def cast(src: torch.Tensor, dst: torch.Tensor):
    """dst = src converted elementwise (fp32 -> fp16/bf16 round-to-nearest-even, 16-bit -> fp32
    exact): the cast of a ppl_copy between tiles of different dtypes."""
    dev = _dev(src, dst)
    _contig("src", src)
    _contig("dst", dst)
    if src.numel() != dst.numel():
        raise ValueError("src and dst must have the same number of elements")
    lib.call("tlm_cast", _ptr(src), dtype_code(src.dtype), _ptr(dst), dtype_code(dst.dtype),
             src.numel(), _stream(dev))
    return dst


def _as_operand(t: torch.Tensor, dt: Optional[torch.dtype]) -> torch.Tensor:
    """t itself, or a device copy rounded to the matrix-operand dtype dt (fp32 programs that copy
    their tiles to fp16 before ppl_gemm); the copy is made by the tlm_cast kernel."""
    if dt is None or t.dtype == dt:
        return t
    out = torch.empty(t.shape, dtype=dt, device=t.device)
    return cast(t, out)


def gemm(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, trans_b: bool = False,
         operand_dtype: Optional[torch.dtype] = None):
    """c = a @ b (trans_b=False, b [K,N]) or a @ b.T (trans_b=True, b [N,K]); fp32 accumulate.
    operand_dtype: fp32 a/b are first rounded to this 16-bit type."""
    dev = _dev(a, b, c)
    a = _as_operand(a, operand_dtype)
    b = _as_operand(b, operand_dtype)
    for n, t in (("A", a), ("B", b), ("C", c)):
        _contig(n, t)
    M, K = a.shape
    N = b.shape[0] if trans_b else b.shape[1]
    kb = b.shape[1] if trans_b else b.shape[0]
    if kb != K or tuple(c.shape) != (M, N):
        raise ValueError(f"shape mismatch A{tuple(a.shape)} B{tuple(b.shape)} C{tuple(c.shape)}")
    if a.dtype != b.dtype:
        raise ValueError("A and B must share a dtype")
    fn = "tlm_gemm_fp8" if a.dtype in _FP8 else "tlm_gemm"
    lib.call(fn, _ptr(a), _ptr(b), _ptr(c), M, N, K, dtype_code(a.dtype), dtype_code(c.dtype),
             1 if trans_b else 0, _stream(dev))
    return c


def flash_attn_fwd(q, k, v, o, causal: bool, sm_scale: float,
                   operand_dtype: Optional[torch.dtype] = None):
    """BSHD attention forward: q, o [B, S, H, D]; k, v [B, S, H_kv, D] with H % H_kv == 0
    (grouped-query attention when H_kv < H). o may be fp32 with 16-bit q/k/v; operand_dtype:
    fp32 q/k/v are first rounded to this 16-bit type (the fp32 program)."""
    dev = _dev(q, k, v, o)
    for n, t in (("Q", q), ("K", k), ("V", v), ("O", o)):
        _contig(n, t)
    if q.dim() != 4 or q.shape != o.shape or k.shape != v.shape or k.dim() != 4:
        raise ValueError("Q, O must be [B, S, H, D] and K, V [B, S, H_kv, D]")
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    if (k.shape[0], k.shape[1], k.shape[3]) != (B, S, D) or Hkv == 0 or H % Hkv:
        raise ValueError(f"K/V {tuple(k.shape)} do not match Q {tuple(q.shape)} "
                         "(same B, S, D; H a multiple of H_kv)")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("Q, K and V must share a dtype")
    q, k, v = (_as_operand(t, operand_dtype) for t in (q, k, v))
    if o.dtype not in (q.dtype, torch.float32):
        raise ValueError(f"O must be {q.dtype} or float32")
    lib.call("tlm_flash_attn_fwd_ex", _ptr(q), _ptr(k), _ptr(v), _ptr(o), B, S, H, Hkv, D,
             1 if causal else 0, float(sm_scale), dtype_code(q.dtype), dtype_code(o.dtype),
             _stream(dev))
    return o


def flash_attn_bhsd_fwd(q, k, v, o, causal: bool, sm_scale: float):
    """BHSD attention forward: q, o [B, H, S_q, D]; k, v [B, H_kv, S_kv, D] with H % H_kv == 0.
    S_q and S_kv may differ; causal keeps key j <= i + S_kv - S_q for query i."""
    dev = _dev(q, k, v, o)
    for n, t in (("Q", q), ("K", k), ("V", v), ("O", o)):
        _contig(n, t)
    if q.dim() != 4 or q.shape != o.shape or k.shape != v.shape or k.dim() != 4:
        raise ValueError("Q, O must be [B, H, S_q, D] and K, V [B, H_kv, S_kv, D]")
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    if (k.shape[0], k.shape[3]) != (B, D) or Hkv == 0 or H % Hkv:
        raise ValueError(f"K/V {tuple(k.shape)} do not match Q {tuple(q.shape)} "
                         "(same B, D; H a multiple of H_kv)")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("Q, K and V must share a dtype")
    if o.dtype not in (q.dtype, torch.float32):
        raise ValueError(f"O must be {q.dtype} or float32")
    lib.call("tlm_flash_attn_bhsd_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(o), B, H, Hkv, Sq, Sk, D,
             1 if causal else 0, float(sm_scale), dtype_code(q.dtype), dtype_code(o.dtype),
             _stream(dev))
    return o


def flash_attn_varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, o,
                          causal: bool, sm_scale: float):
    """Attention over unpadded sequences: q, o [total_q, H, D]; k, v [total_k, H_kv, D];
    sequence b is rows cu_seqlens_q[b] .. cu_seqlens_q[b + 1] of q (int32 [B + 1]) and the
    matching rows of k, v. Queries at positions >= max_seqlen_q are not computed."""
    dev = _dev(q, k, v, o, cu_seqlens_q, cu_seqlens_k)
    for n, t in (("Q", q), ("K", k), ("V", v), ("O", o), ("cu_seqlens_q", cu_seqlens_q),
                 ("cu_seqlens_k", cu_seqlens_k)):
        _contig(n, t)
    if q.dim() != 3 or q.shape != o.shape or k.shape != v.shape or k.dim() != 3:
        raise ValueError("Q, O must be [total_q, H, D] and K, V [total_k, H_kv, D]")
    total_q, H, D = q.shape
    total_k, Hkv = k.shape[0], k.shape[1]
    if k.shape[2] != D or Hkv == 0 or H % Hkv:
        raise ValueError(f"K/V {tuple(k.shape)} do not match Q {tuple(q.shape)} "
                         "(same D; H a multiple of H_kv)")
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32 or \
            cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape != cu_seqlens_k.shape or \
            cu_seqlens_q.numel() < 1:
        raise ValueError("cu_seqlens_q / cu_seqlens_k must be int32 [B + 1]")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("Q, K and V must share a dtype")
    if o.dtype not in (q.dtype, torch.float32):
        raise ValueError(f"O must be {q.dtype} or float32")
    B = cu_seqlens_q.numel() - 1
    lib.call("tlm_flash_attn_varlen_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(o),
             _ptr(cu_seqlens_q), _ptr(cu_seqlens_k), B, int(max_seqlen_q), total_q, total_k, H,
             Hkv, D, 1 if causal else 0, float(sm_scale), dtype_code(q.dtype),
             dtype_code(o.dtype), _stream(dev))
    return o


def flash_attn_splitkv_workspace_bytes(B, S_q, S_kv, H, D, num_split) -> int:
    return int(lib.load().tlm_flash_attn_splitkv_workspace_bytes(B, S_q, S_kv, H, D, num_split))


def flash_attn_splitkv_fwd(q, k, v, glse, o_partial, o, num_split: int, sm_scale: float,
                           workspace: torch.Tensor):
    """Split-KV inference attention (example_mha_inference.py): q, o [B, S_q, H, D]; k, v
    [B, S_kv, H_kv, D]; writes glse [B, H, num_split, S_q], o_partial [B, S_q, H, num_split, D]
    (each split's log2 sum-exp and normalised output, rounded to the dtype) and o, their
    combine."""
    dev = _dev(q, k, v, glse, o_partial, o, workspace)
    for n, t in (("Q", q), ("K", k), ("V", v), ("glse", glse), ("Output_partial", o_partial),
                 ("Output", o), ("workspace", workspace)):
        _contig(n, t)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape or o.shape != q.shape:
        raise ValueError("Q, Output must be [B, S_q, H, D] and K, V [B, S_kv, H_kv, D]")
    B, Sq, H, D = q.shape
    Skv, Hkv = k.shape[1], k.shape[2]
    if k.shape[0] != B or k.shape[3] != D or Hkv == 0 or H % Hkv:
        raise ValueError(f"K/V {tuple(k.shape)} do not match Q {tuple(q.shape)}")
    if tuple(glse.shape) != (B, H, num_split, Sq) or \
            tuple(o_partial.shape) != (B, Sq, H, num_split, D):
        raise ValueError("glse must be [B, H, num_split, S_q] and Output_partial "
                         "[B, S_q, H, num_split, D]")
    if len({q.dtype, k.dtype, v.dtype, glse.dtype, o_partial.dtype, o.dtype}) != 1:
        raise ValueError("all tensors must share one 16-bit dtype")
    ws_bytes = workspace.numel() * workspace.element_size()
    lib.call("tlm_flash_attn_splitkv_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(glse),
             _ptr(o_partial), _ptr(o), _ptr(workspace), ws_bytes, B, Sq, Skv, H, Hkv, D,
             int(num_split), float(sm_scale), dtype_code(q.dtype), _stream(dev))
    return o


def sigmoid(x: torch.Tensor, y: torch.Tensor):
    """y = sigmoid(x), fp32 math."""
    dev = _dev(x, y)
    _contig("x", x)
    _contig("y", y)
    if x.shape != y.shape or x.dtype != y.dtype:
        raise ValueError("x and y must share shape and dtype")
    lib.call("tlm_sigmoid", _ptr(x), _ptr(y), x.numel(), dtype_code(x.dtype), _stream(dev))
    return y


def gather_rows(param: torch.Tensor, index: torch.Tensor, out: torch.Tensor):
    """out[i, :] = param[index[i], :] (index uint32 or int32, read as unsigned; an index past the
    last row gives a zero row)."""
    dev = _dev(param, index, out)
    for n, t in (("param", param), ("index", index), ("out", out)):
        _contig(n, t)
    if param.dim() != 2 or out.dim() != 2 or out.shape[1] != param.shape[1]:
        raise ValueError("param [rows, H] and out [n, H] must share H")
    if index.dtype not in (torch.int32, torch.uint32) or index.numel() != out.shape[0]:
        raise ValueError("index must hold one int32 / uint32 per output row")
    if out.dtype != param.dtype:
        raise ValueError("out must have param's dtype")
    lib.call("tlm_gather_rows", _ptr(param), param.shape[0], param.shape[1] * param.element_size(),
             _ptr(index), index.numel(), _ptr(out), _stream(dev))
    return out


def topk(src: torch.Tensor, k: int, descending: bool, values: torch.Tensor,
         indices: torch.Tensor):
    """Sort src (1-D) with its indices into values / indices; the first k are the top k."""
    dev = _dev(src, values, indices)
    for n, t in (("src", src), ("values", values), ("indices", indices)):
        _contig(n, t)
    L = src.numel()
    if values.numel() != L or indices.numel() != L or values.dtype != src.dtype:
        raise ValueError("values and indices must have src's length (and values its dtype)")
    if indices.dtype != torch.int32:
        raise ValueError("indices must be int32")
    lib.call("tlm_topk", _ptr(src), L, int(k), 1 if descending else 0, dtype_code(src.dtype),
             _ptr(values), _ptr(indices), _stream(dev))
    return values, indices


def row_reduce(x: torch.Tensor, y: torch.Tensor, op: str):
    """y[r] = max / sum over the last dim of x (op "max" or "sum")."""
    dev = _dev(x, y)
    _contig("x", x)
    _contig("y", y)
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    if y.numel() != rows:
        raise ValueError(f"y must hold one value per row ({rows})")
    code = {"max": lib.REDUCE_MAX, "sum": lib.REDUCE_SUM}[op]
    lib.call("tlm_row_reduce", _ptr(x), _ptr(y), rows, cols, code, dtype_code(x.dtype),
             dtype_code(y.dtype), _stream(dev))
    return y


def mla_workspace_bytes(B, Hq, dv, num_split) -> int:
    return int(lib.load().tlm_mla_workspace_bytes(B, Hq, dv, num_split))


def _rows(name, t, width):
    """Row pointer and row stride (elements) of a [..., width] tensor whose last dim is dense."""
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: last dim must be contiguous")
    if t.shape[-1] != width:
        raise ValueError(f"{name}: last dim must be {width}, got {t.shape[-1]}")
    # every leading dim must collapse onto one row stride
    rs = None
    expect = None
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] == 1:
            continue
        if rs is None:
            rs = t.stride(d)
            expect = rs * t.shape[d]
        else:
            if t.stride(d) != expect:
                raise ValueError(f"{name}: leading dims do not form uniform rows")
            expect = t.stride(d) * t.shape[d]
    return t.data_ptr(), (rs if rs is not None else width)


def _rows_count(kv, dv, k_pe, dpe) -> int:
    """Token rows addressable in both the latent and the rope views of the cache."""
    return min(kv.numel() // dv, k_pe.numel() // dpe)


def mla_decode(q, q_pe, kv, k_pe, block_table, seqlens, out, workspace, page: int,
               num_split: int, sm_scale: float, kv_scale: Optional[torch.Tensor] = None,
               glse: Optional[torch.Tensor] = None, o_partial: Optional[torch.Tensor] = None,
               part_block: int = 64):
    """Paged MLA decode. q [B,Hq,dv], q_pe [B,Hq,dpe], kv [rows,...,dv], k_pe [rows,...,dpe]
    (any uniform row stride), block_table int32 [B, max_pages], seqlens int32 [B],
    out [B, Hq, dv]. kv_scale: device fp32 scalar for fp8 KV (None -> 1). glse [B, Hq, ns] and
    o_partial [B, Hq, ns, dv] (both or neither): the split programs' partials, written over
    the program's partition in blocks of part_block tokens."""
    dev = _dev(q, q_pe, kv, k_pe, block_table, seqlens, out, workspace, kv_scale, glse,
               o_partial)
    B, Hq, dv = q.shape
    dpe = q_pe.shape[-1]
    if tuple(q_pe.shape[:2]) != (B, Hq) or tuple(out.shape) != (B, Hq, dv):
        raise ValueError("q_pe/out shapes do not match q")
    q_ptr, q_rs = _rows("Q", q, dv)
    qpe_ptr, qpe_rs = _rows("Q_pe", q_pe, dpe)
    if q_rs % 1 or q.stride(1) != q_rs or q_pe.stride(1) != qpe_rs:
        raise ValueError("Q/Q_pe rows must be uniform over (batch, head)")
    kv_ptr, kv_rs = _rows("KV", kv, dv)
    kpe_ptr, kpe_rs = _rows("K_pe", k_pe, dpe)
    _contig("block_table", block_table)
    _contig("cache_seqlens", seqlens)
    _contig("Output", out)
    if block_table.dtype != torch.int32 or seqlens.dtype != torch.int32:
        raise ValueError("block_table and cache_seqlens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or seqlens.numel() != B:
        raise ValueError("block_table must be [B, max_pages] and cache_seqlens [B]")
    if q.dtype != q_pe.dtype or kv.dtype != k_pe.dtype:
        raise ValueError("Q/Q_pe and KV/K_pe must share dtypes")
    if kv.dtype == torch.float8_e4m3fn:
        if kv_scale is None:
            raise ValueError("fp8 KV needs a kv_scale tensor")
    if kv_scale is not None and (kv_scale.dtype != torch.float32 or kv_scale.numel() != 1):
        raise ValueError("kv_scale must be a one-element float32 tensor")
    ws_bytes = workspace.numel() * workspace.element_size()
    if (glse is None) != (o_partial is None):
        raise ValueError("glse and Output_partial go together")
    if glse is None:
        lib.call("tlm_mla_decode", q_ptr, qpe_ptr, q_rs, qpe_rs, kv_ptr, kpe_ptr, kv_rs, kpe_rs,
                 _rows_count(kv, dv, k_pe, dpe), _ptr(block_table), _ptr(seqlens), _ptr(out),
                 _ptr(workspace), ws_bytes, B, Hq, dv, dpe, page, block_table.shape[1],
                 num_split, float(sm_scale), _ptr(kv_scale), dtype_code(q.dtype),
                 dtype_code(kv.dtype), dtype_code(out.dtype), _stream(dev))
        return out
    _contig("glse", glse)
    _contig("Output_partial", o_partial)
    if tuple(glse.shape) != (B, Hq, num_split) or \
            tuple(o_partial.shape) != (B, Hq, num_split, dv) or glse.dtype != o_partial.dtype:
        raise ValueError("glse must be [B, Hq, num_split] and Output_partial [B, Hq, num_split, "
                         "dv], of one dtype")
    lib.call("tlm_mla_decode_ex", q_ptr, qpe_ptr, q_rs, qpe_rs, kv_ptr, kpe_ptr, kv_rs, kpe_rs,
             _rows_count(kv, dv, k_pe, dpe), _ptr(block_table), _ptr(seqlens), _ptr(out),
             _ptr(workspace), ws_bytes, B, Hq, dv, dpe, page, block_table.shape[1], num_split,
             float(sm_scale), _ptr(kv_scale), dtype_code(q.dtype), dtype_code(kv.dtype),
             dtype_code(out.dtype), _ptr(glse), _ptr(o_partial), int(part_block),
             dtype_code(glse.dtype), _stream(dev))
    return out


def paged_gather(kv_bytes: torch.Tensor, block_table, seqlens, cu_seqlens, out, page: int):
    """Bit-exact gather of every sequence's token rows through the block table."""
    dev = _dev(kv_bytes, block_table, seqlens, cu_seqlens, out)
    row_bytes = kv_bytes.shape[-1] * kv_bytes.element_size()
    kv_rows = kv_bytes.numel() * kv_bytes.element_size() // row_bytes
    lib.call("tlm_paged_gather", _ptr(kv_bytes), row_bytes, kv_rows, _ptr(block_table),
             _ptr(seqlens),
             _ptr(cu_seqlens), _ptr(out), block_table.shape[0], page, block_table.shape[1],
             _stream(dev))
    return out


def kv_append_fp8(x: torch.Tensor, start: torch.Tensor, count: torch.Tensor,
                  block_table: torch.Tensor, kv: torch.Tensor, page: int, scale: torch.Tensor):
    """Quantise new latent rows x [B, T, D] (bf16/fp16) to e4m3 with the cache scale and write
    them into the paged fp8 pool kv [rows, D] at positions start[b] .. start[b] + count[b] - 1
    of each sequence (saturating at +-448). Returns kv."""
    dev = _dev(x, start, count, block_table, kv, scale)
    if x.dim() != 3:
        raise ValueError("x must be [B, T, D]")
    B, T, D = x.shape
    if x.stride(2) != 1:
        raise ValueError("x rows must be contiguous")
    if kv.dtype != torch.float8_e4m3fn or kv.dim() != 2 or kv.shape[1] != D or kv.stride(1) != 1:
        raise ValueError("kv must be a float8_e4m3fn [rows, D] tensor with contiguous rows")
    for n, t in (("start", start), ("count", count), ("block_table", block_table)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{n} must be a contiguous int32 tensor")
    if start.numel() != B or count.numel() != B or block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError("start/count must have B entries and block_table B rows")
    if scale.dtype != torch.float32 or scale.numel() != 1:
        raise ValueError("scale must be a one-element float32 tensor")
    lib.call("tlm_kv_append_fp8", _ptr(x), x.stride(0), x.stride(1), dtype_code(x.dtype),
             _ptr(start), _ptr(count), _ptr(block_table), block_table.shape[1], page, _ptr(kv),
             kv.stride(0), kv.shape[0], B, T, D, _ptr(scale), _stream(dev))
    return kv


def elementwise(inputs, bcast, outputs, code, consts, rows: int, cols: int):
    """Run an elementwise register program (include/tlmi355x.h: tlm_elementwise) over the
    [rows, cols] output domain. inputs: tensors (F32 / F16 / BF16) with their broadcast kinds
    (lib.EW_FULL, EW_ROW for an [rows, 1] tensor, EW_COL, EW_SCALAR); outputs: tensors of
    rows * cols elements; code: instruction words; consts: fp32 constants."""
    import ctypes
    dev = _dev(*inputs, *outputs)
    for t in list(inputs) + list(outputs):
        _contig("operand", t)
    for t in outputs:
        if t.numel() != rows * cols:
            raise ValueError(f"output of {t.numel()} elements for a {rows} x {cols} domain")
    if len(bcast) != len(inputs):
        raise ValueError("one broadcast kind per input")
    need = {lib.EW_FULL: rows * cols, lib.EW_ROW: rows, lib.EW_COL: cols, lib.EW_SCALAR: 1}
    for t, bc in zip(inputs, bcast):
        if bc not in need or t.numel() < need[bc]:
            raise ValueError(f"input of {t.numel()} elements for broadcast kind {bc} over a "
                             f"{rows} x {cols} domain")
    n_in, n_out = len(inputs), len(outputs)
    P, I = ctypes.c_void_p, ctypes.c_int
    in_p = (P * max(1, n_in))(*[t.data_ptr() for t in inputs])
    in_dt = (I * max(1, n_in))(*[dtype_code(t.dtype) for t in inputs])
    in_bc = (I * max(1, n_in))(*bcast)
    out_p = (P * n_out)(*[t.data_ptr() for t in outputs])
    out_dt = (I * n_out)(*[dtype_code(t.dtype) for t in outputs])
    cw = (ctypes.c_int32 * len(code))(*[(c if c < 2 ** 31 else c - 2 ** 32) for c in code])
    cf = (ctypes.c_float * max(1, len(consts)))(*consts)
    lib.call("tlm_elementwise", in_p, in_dt, in_bc, n_in, out_p, out_dt, n_out, cw, len(code),
             cf, len(consts), int(rows), int(cols), _stream(dev))
    return outputs
