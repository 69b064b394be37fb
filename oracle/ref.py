"""CPU oracle: restatements of the reference's own torch reference functions for the kernel path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this module, as the checker / CPU baseline — never as the thing measured or shipped.
The product path (tilelang -> libtlmi355x.so) never imports it and has no CPU fallback.

Each function cites the reference file:line it restates. Stated deviations from the reference
(all listed in the module-level notes of each function) follow the benchmark configs:
  * rmsnorm: weight and eps are parameters (the demo has no weight and eps 1e-12);
  * rope tables are computed in fp32 then cast (the demo computes angles in bf16, which cannot
    represent positions > 256 exactly) and the rotation is evaluated in fp32 with one rounding;
  * flash attention causal masking is the element mask of ref_program (tril);
  * mla gathers tokens through the block table (the reference oracle assumes an identity
    table, begin = i*max_seqlen_pad) and dequantises fp8 KV with a per-tensor scale.

How each function is pinned (checks that do not retype the formula) is in tests/test_oracle.py.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

LOG2E_REF = 1.44269504  # constant used by the reference's MLA programs (example_mla_decode_paged.py:12)


# ------------------------------------------------------------------------------------------------
# RMSNorm — tpu_demo/rms_norm/rms_norm_fp16.py:51-54:
#   ref_fp32 = a_fp32 / sqrt(mean(a_fp32*a_fp32, dim=1, keepdim=True) + eps); ref = ref_fp32.to(dtype)
def rmsnorm_ref(x: torch.Tensor, w: Optional[torch.Tensor] = None, eps: float = 1e-12):
    xf = x.float()
    y = xf / torch.sqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


# ------------------------------------------------------------------------------------------------
# GEMM — tpu_demo/matmul/tpu_test_matmul_fp16.py:45 (ref = torch.matmul(a, b).half()), with the
# fp32 accumulation of the program (ppl_gemm C is fp32, tpu_test_matmul_fp16.py:19-29) and of
# testing/python/amd/test_tilelang_test_amd.py:90-99 (a.float() @ b.float()).
def matmul_ref(a: torch.Tensor, b: torch.Tensor, out_dtype=torch.float16, trans_b=False):
    bf = b.float().t() if trans_b else b.float()
    return (a.float() @ bf).to(out_dtype)


# FP8 GEMM — examples/gemm_fp8/example_tilelang_gemm_fp8.py:46-55: ref = (a.half() @
# b.half().T).to(fp8). fp8 products are exact in fp32, so the product is accumulated in fp32 (not
# fp16, which the example's GPU reference rounds to before the fp8 cast) and rounded once.
def gemm_fp8_ref(a: torch.Tensor, b_nk: torch.Tensor, out_dtype=torch.float32):
    return (a.float() @ b_nk.float().t()).to(out_dtype)


# ------------------------------------------------------------------------------------------------
# Remaining TPU demo ops.
# sigmoid — tpu_demo/tpu_test_sigmoid_fp32.py:48 (ref = torch.sigmoid(a)), fp32, one rounding.
def sigmoid_ref(x: torch.Tensor) -> torch.Tensor:
    return torch.sigmoid(x.float()).to(x.dtype)


# gather — tpu_demo/tpu_test_gather_fp32.py:38 (ref = param[idx]); indices read as uint32, an
# index past the last row gives a zero row (the kernel's stated choice).
def gather_ref(param: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    idx = index.reshape(-1).to(torch.int64) & 0xFFFFFFFF
    out = torch.zeros(idx.numel(), param.shape[1], dtype=param.dtype)
    ok = idx < param.shape[0]
    out[ok] = param[idx[ok]]
    return out


# topk — tpu_demo/tpu_test_topk_fp32.py:36 (torch.topk(src, K, largest=True, sorted=True)); the
# HAU sort writes the whole vector in order (codegen_ppl.cc:1878-1907). Full order: a stable sort
# by value (NaN above every number, -0.0 == +0.0), ties by index.
def topk_ref(src: torch.Tensor, descending: bool = True):
    if src.dtype == torch.uint32:
        a = src.view(torch.int32).numpy().view(np.uint32).astype(np.int64)
        order = np.argsort(-a if descending else a, kind="stable")
        return src[torch.from_numpy(order)], torch.from_numpy(order.astype(np.int32))
    vals, idx = torch.sort(src, descending=descending, stable=True)
    return vals, idx.to(torch.int32)


# row reductions — tpu_demo/tpu_test_reduce_max.py:36 (torch.max(x, dim=1, keepdim=True)),
# tpu_test_reduce_sum.py:36 (torch.sum(x, dim=1, keepdim=True)); fp32 accumulation, one rounding.
def row_reduce_ref(x: torch.Tensor, op: str, out_dtype=None) -> torch.Tensor:
    xf = x.float()
    r = xf.max(dim=-1, keepdim=True).values if op == "max" else xf.sum(dim=-1, keepdim=True)
    return r.to(out_dtype or x.dtype)


# Stand-alone elementwise programs (tpu_demo/ppl/test, elementwise_add_kernel), fp32 math with
# one rounding per tile write, as the programs' tile dtypes hold the values.
# exp.py:6-16 / exp_bf16.py: in-place ppl_exp2 (natural exponential, customize.py:313-339).
def ppl_exp_ref(x: torch.Tensor) -> torch.Tensor:
    return torch.exp(x.float()).to(x.dtype)


# mul_N_1.py:9-22: C = A * B, B [M, 1] broadcast along each row (codegen_ppl.cc:874-883).
def ppl_mul_rows_ref(a: torch.Tensor, b_col: torch.Tensor) -> torch.Tensor:
    return (a.float() * b_col.float().reshape(-1, 1)).to(a.dtype)


# elementwise_c.py:9-22: B = A * C1 + C2 (ppl_mul_C, then ppl_add_C; the tile holds the product).
def ppl_scale_shift_ref(a: torch.Tensor, scale: float, shift: float) -> torch.Tensor:
    t = (a.float() * scale).to(a.dtype).float()
    return (t + shift).to(a.dtype)


# elementwise_add.py:37-38 (ref_add = torch.add(a, b)), cast to C's dtype.
def ppl_add_ref(a: torch.Tensor, b: torch.Tensor, out_dtype=None) -> torch.Tensor:
    return (a.float() + b.float()).to(out_dtype or a.dtype)


# ------------------------------------------------------------------------------------------------
# RoPE — tables per tpu_demo/tpu_test_rope_bf16.py:53-74 (make_rope_cos_sin), computed in fp32;
# rotation as the program computes it: ppl_rope_add (codegen_ppl.cc:1809-1848: out[2i] =
# e1[2i] + e2[2i+1], out[2i+1] = o1[2i+1] + o2[2i]) over the tiles x*cos, -x*sin, x*cos, x*sin
# (tpu_test_rope_bf16.py:28-45). With the demo's paired tables (cos[2i] = cos[2i+1], sin alike)
# this is rope_ref_torch (:76-92).
def rope_cos_sin(C: int, W: int, base: float = 10000.0, pos_start: int = 0,
                 dtype=torch.bfloat16):
    assert W % 2 == 0
    k = torch.arange(W // 2, dtype=torch.float32)
    inv_freq = base ** (-2.0 * k / W)
    pos = torch.arange(pos_start, pos_start + C, dtype=torch.float32).unsqueeze(1)
    theta = pos * inv_freq
    c, s = torch.cos(theta), torch.sin(theta)
    cos = torch.repeat_interleave(c, 2, dim=1)
    sin = torch.repeat_interleave(s, 2, dim=1)
    return cos.to(dtype).contiguous(), sin.to(dtype).contiguous()


def rope_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., tokens?, W] with cos/sin broadcastable as [tokens, 1.., W] (or x's shape)."""
    xf, cf, sf = x.float(), cos.float(), sin.float()
    if cf.shape != xf.shape:  # tables [T, W] shared across heads of x [T, H, W]
        cf = cf.view(cf.shape[0], *([1] * (xf.dim() - 2)), cf.shape[-1])
        sf = sf.view(sf.shape[0], *([1] * (xf.dim() - 2)), sf.shape[-1])
    xe, xo = xf[..., 0::2], xf[..., 1::2]
    ce, co = cf[..., 0::2], cf[..., 1::2]
    se, so = sf[..., 0::2], sf[..., 1::2]
    out = torch.empty_like(xf.expand(*torch.broadcast_shapes(xf.shape, cf.shape)))
    out[..., 0::2] = xe * ce - xo * so
    out[..., 1::2] = xo * co + xe * se
    return out.to(x.dtype)


# ------------------------------------------------------------------------------------------------
# SwiGLU — tpu_demo/tpu_test_swiglu_bf16.py:68: ref = b * F.silu(a), evaluated in fp32 (the
# program computes in fp32, :37-52) with one rounding.
def swiglu_ref(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return (up.float() * F.silu(gate.float())).to(gate.dtype)


def mlp_ref(x, gate_weight, up_weight, down_weight, operand_dtype=None):
    """tpu_demo/ppl/mlp/mlp_bf16.py:98-131 with whole blocks: gate = x Wg^T and up = x Wu^T
    (fp32 accumulation, stored as the 16-bit dtype), SiLU(gate) * up in fp32 rounded to the
    16-bit dtype, out = gated Wd^T (fp32 accumulation, 16-bit result). mlp_fp32.py:83-120
    (operand_dtype bf16): the fp32 x and weights are first rounded to the operand dtype, and
    the 16-bit down projection is returned as fp32."""
    dt = operand_dtype or x.dtype
    x, gate_weight, up_weight, down_weight = (v.to(dt) for v in
                                              (x, gate_weight, up_weight, down_weight))
    gate = (x.float() @ gate_weight.float().t()).to(dt)
    up = (x.float() @ up_weight.float().t()).to(dt)
    g = gate.float()
    h = (g / (1.0 + torch.exp(-g)) * up.float()).to(dt)
    out = (h.float() @ down_weight.float().t()).to(dt)
    return out if operand_dtype is None else out.float()


# ------------------------------------------------------------------------------------------------
# FlashAttention — tpu_demo/flashattn/tpu_test_flashattn_bf16.py:171-182 (ref_program):
#   scores = einsum('bqhd,bkhd->bhqk', Q.float(), K.float()) / sqrt(dim); causal tril mask;
#   softmax; out = einsum('bhqk,bkhd->bqhd', P, V.float()).bfloat16()
# Evaluated one (batch, head) at a time so the [S, S] scores fit in host memory.
def flashattn_ref(Q, K, V, causal: bool, sm_scale: Optional[float] = None,
                  heads: Optional[list] = None, batches: Optional[list] = None):
    """K, V may have fewer heads than Q (grouped-query attention): query head h reads K/V head
    h // (H // H_kv), as examples/flash_attention/example_gqa_fwd_bshd.py:181-205 (ref_program:
    K.repeat_interleave(groups, dim=2))."""
    B, S, H, D = Q.shape
    G = H // K.shape[2]
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    out = torch.empty(B, S, H, D, dtype=torch.float32)
    mask = None
    if causal:
        mask = torch.ones(S, S, dtype=torch.bool).tril()
    bs = range(B) if batches is None else batches
    hs = range(H) if heads is None else heads
    for b in bs:
        for h in hs:
            q = Q[b, :, h, :].float()
            k = K[b, :, h // G, :].float()
            v = V[b, :, h // G, :].float()
            s = (q @ k.t()) * scale
            if mask is not None:
                s = s.masked_fill(~mask, float("-inf"))
            out[b, :, h, :] = torch.softmax(s, dim=-1) @ v
    return out.to(Q.dtype)


def flashattn_rows_ref(Q, K, V, causal: bool, rows, sm_scale: Optional[float] = None):
    """flashattn_ref restricted to the query positions ``rows`` (every batch and head): the same
    fp32 softmax(Q K^T * scale) V of tpu_test_flashattn_bf16.py:171-182 with the causal tril
    mask, computed per batch for all heads at once. Returns fp32 [B, len(rows), H, D]."""
    B, S, H, D = Q.shape
    G = H // K.shape[2]
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    rows = torch.as_tensor(rows, dtype=torch.long)
    out = torch.empty(B, len(rows), H, D, dtype=torch.float32)
    keep = None
    if causal:
        keep = torch.arange(S)[None, :] <= rows[:, None]  # [R, S]
    for b in range(B):
        q = Q[b, rows].float().permute(1, 0, 2)  # [H, R, D]
        k = K[b].float().repeat_interleave(G, dim=1).permute(1, 2, 0)  # [H, D, S]
        v = V[b].float().repeat_interleave(G, dim=1).permute(1, 0, 2)  # [H, S, D]
        s = torch.bmm(q, k.contiguous()) * scale
        if keep is not None:
            s = s.masked_fill(~keep[None], float("-inf"))
        out[b] = torch.bmm(torch.softmax(s, dim=-1), v.contiguous()).permute(1, 0, 2)
    return out


def flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal: bool = False,
                         sm_scale: Optional[float] = None, max_seqlen_q: Optional[int] = None):
    """Attention over unpadded sequences, examples/flash_attention/example_mha_fwd_varlen.py:
    attention_ref (:166-219) on the padded batch is, per sequence b, fp32 attention of query rows
    cu_q[b] .. cu_q[b + 1] over key rows cu_k[b] .. cu_k[b + 1] (padded keys masked with -inf,
    :206-207; padded query rows zeroed, :214-218); K/V head h // (H // H_kv) as attention_ref's
    repeat (:203-204). q [total_q, H, D], k, v [total_k, H_kv, D]; returns fp32
    [total_q, H, D].
    causal (not exercised by the example, whose attention_ref ignores it) keeps key j <= i +
    nk - nq, the file's construct_local_mask with window (-1, 0) (:156-157). A query that sees no
    key gets zeros (attention_ref's softmax gives NaN there); rows at positions >= max_seqlen_q
    are left as NaN (the kernel does not write them)."""
    total_q, H, D = q.shape
    G = H // k.shape[1]
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    out = torch.full((total_q, H, D), float("nan"), dtype=torch.float32)
    cq, ck = cu_q.tolist(), cu_k.tolist()
    for b in range(len(cq) - 1):
        q0, q1, k0, k1 = cq[b], cq[b + 1], ck[b], ck[b + 1]
        nq, nk = q1 - q0, k1 - k0
        nrow = nq if max_seqlen_q is None else min(nq, max_seqlen_q)
        if nrow <= 0:
            continue
        for h in range(H):
            qq = q[q0:q0 + nrow, h, :].float()
            kk = k[k0:k1, h // G, :].float()
            vv = v[k0:k1, h // G, :].float()
            s = (qq @ kk.t()) * scale
            if causal:
                i = torch.arange(nrow).view(-1, 1)
                j = torch.arange(nk).view(1, -1)
                s = s.masked_fill(j > i + (nk - nq), float("-inf"))
            seen = torch.isfinite(s).any(dim=1, keepdim=True)
            p = torch.softmax(s, dim=-1).nan_to_num(0.0) if nk > 0 else s
            o = p @ vv if nk > 0 else torch.zeros(nrow, D)
            out[q0:q0 + nrow, h, :] = torch.where(seen, o, torch.zeros_like(o))
    return out


def flashattn_bhsd_ref(Q, K, V, causal: bool, sm_scale: Optional[float] = None):
    """Head-major attention, examples/flash_attention/example_mha_fwd_bhsd.py ref_program
    (:175-188): fp32 scores Q K^T / sqrt(dim) per (batch, head), softmax over keys, times V.
    Q [B, H, S_q, D]; K, V [B, H_kv, S_kv, D] (query head h reads K/V head h // (H // H_kv)).
    causal keeps key j <= i + S_kv - S_q, the kernel's mask (q_idx = bx * block_M + i + past_len,
    :50-55); ref_program's torch.tril(ones(seq_q, seq_kv)) is the same set when S_q == S_kv, the
    only case in which the example's loop bound agrees with its mask. A query that sees no key
    gets zeros. Returns fp32 [B, H, S_q, D]."""
    B, H, Sq, D = Q.shape
    Sk = K.shape[2]
    G = H // K.shape[1]
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else sm_scale
    out = torch.zeros(B, H, Sq, D, dtype=torch.float32)
    if Sk == 0:
        return out
    keep = None
    if causal:
        keep = torch.arange(Sk).view(1, -1) <= torch.arange(Sq).view(-1, 1) + (Sk - Sq)
    for b in range(B):
        for h in range(H):
            s = (Q[b, h].float() @ K[b, h // G].float().t()) * scale
            if keep is not None:
                s = s.masked_fill(~keep, float("-inf"))
            p = torch.softmax(s, dim=-1).nan_to_num(0.0)  # rows without a key: all -inf -> 0
            out[b, h] = p @ V[b, h // G].float()
    return out


# ------------------------------------------------------------------------------------------------
# Split-KV inference attention — examples/flash_attention/example_mha_inference.py
def mha_inference_ref(Q, K, V, sm_scale: Optional[float] = None):
    """examples/flash_attention/example_mha_inference.py ref_program (:206-213): sequence-major
    Q [B, S_q, H, D], K, V [B, S_kv, H, D], fp32 softmax(Q K^T / sqrt(D)) V over all keys (the
    program is non-causal). Returns fp32 [B, S_q, H, D]."""
    o = flashattn_bhsd_ref(Q.permute(0, 2, 1, 3), K.permute(0, 2, 1, 3), V.permute(0, 2, 1, 3),
                           False, sm_scale)
    return o.permute(0, 2, 1, 3).contiguous()


def mha_split_combine_ref(Q, K, V, num_split: int, block_N: int, store_dtype=torch.float16):
    """The split-KV algorithm of example_mha_inference.py (flash_split_ref :230-275, reduce_ref
    :216-227): each split s covers keys [s per, (s + 1) per), per = S_kv // num_split, in tiles of
    block_N with the online softmax in the exp2 domain; its normalised output and
    lse = log2(l) + m * scale are stored in store_dtype (the program's glse / Output_partial);
    the merge weights each split by 2^(lse_s - log2 sum_s 2^lse_s). Returns fp32 [B, S_q, H, D]
    and the stored (glse [B, H, num_split, S_q], partial [B, S_q, H, num_split, D])."""
    B, Sq, H, D = Q.shape
    Skv = K.shape[1]
    per = Skv // num_split
    scale = (1.0 / D) ** 0.5 * 1.44269504
    q = Q.float() * scale
    glse = torch.empty(B, H, num_split, Sq, dtype=torch.float32)
    part = torch.empty(B, Sq, H, num_split, D, dtype=torch.float32)
    for s in range(num_split):
        m = torch.full((B, H, Sq), float("-inf"))
        l = torch.zeros(B, H, Sq)
        o = torch.zeros(B, Sq, H, D)
        for t in range(per // block_N):
            k0 = s * per + t * block_N
            kk = K[:, k0:k0 + block_N].float()
            vv = V[:, k0:k0 + block_N].float()
            sc = torch.einsum("bqhd,bkhd->bhqk", q, kk)
            m_prev, m = m, torch.maximum(m, sc.amax(-1))
            alpha = torch.exp2(m_prev - m)
            p = torch.exp2(sc - m[..., None])
            l = l * alpha + p.sum(-1)
            o = o * alpha.permute(0, 2, 1)[..., None] + torch.einsum(
                "bhqk,bkhd->bqhd", p.to(Q.dtype).float(), vv)
        o = o / l.permute(0, 2, 1)[..., None]
        glse[:, :, s] = torch.log2(l) + m
        part[:, :, :, s] = o
    glse = glse.to(store_dtype).float()
    part = part.to(store_dtype).float()
    lmax = glse.amax(2)
    lsum = torch.log2(torch.exp2(glse - lmax[:, :, None]).sum(2)) + lmax
    out = torch.zeros(B, Sq, H, D)
    for s in range(num_split):
        w = torch.exp2(glse[:, :, s] - lsum)  # [B, H, S_q]
        out += part[:, :, :, s] * w.permute(0, 2, 1)[..., None]
    return out, (glse, part)


# ------------------------------------------------------------------------------------------------
# MLA decode — examples/deepseek_mla/example_mla_decode_paged.py:259-308 (run_torch_mla /
# scaled_dot_product_attention): per sequence, fp32 attention of q [h_q, d] over the sequence's
# KV rows, shared latent head (h_kv = 1), value = first dv columns of the key rows.
# The rows are gathered through the block table: token j -> BT[b, j // page] * page + j % page
# (the kernel's addressing, :62-63, 147-148). fp8 KV is dequantised as decode(byte) * kv_scale.
def paged_rows(block_table: torch.Tensor, seqlen: int, b: int, page: int) -> torch.Tensor:
    j = torch.arange(seqlen, dtype=torch.int64)
    return block_table[b, j // page].to(torch.int64) * page + j % page


def mla_decode_ref(q, q_pe, kv, k_pe, block_table, seqlens, page: int, sm_scale: float,
                   kv_scale: float = 1.0, out_dtype=torch.bfloat16, return_lse=False):
    """q [B,Hq,dv], q_pe [B,Hq,dpe], kv [rows,dv] / k_pe [rows,dpe] (any dtype incl. fp8),
    block_table int32 [B,P], seqlens int32 [B]. Returns [B,Hq,dv] (and lse [B,Hq], natural log)."""
    B, Hq, dv = q.shape
    kv2 = kv.reshape(kv.shape[0], -1)
    kp2 = k_pe.reshape(k_pe.shape[0], -1)
    out = torch.empty(B, Hq, dv, dtype=torch.float32)
    lse = torch.empty(B, Hq, dtype=torch.float32)
    for b in range(B):
        L = int(seqlens[b])
        rows = paged_rows(block_table, L, b, page)
        vb = kv2[rows].float() * kv_scale  # gather, then dequantise
        kb = torch.cat([vb, kp2[rows].float() * kv_scale], dim=1)  # [L, dv+dpe]
        qb = torch.cat([q[b].float(), q_pe[b].float()], dim=1)  # [Hq, dv+dpe]
        s = (qb @ kb.t()) * sm_scale
        lse[b] = torch.logsumexp(s, dim=-1)
        out[b] = torch.softmax(s, dim=-1) @ vb
    o = out.to(out_dtype)
    return (o, lse) if return_lse else o


def mla_decode_nopage_ref(q, q_pe, kv, k_pe, sm_scale: Optional[float] = None,
                          out_dtype=None):
    """Non-paged MLA decode, examples/deepseek_mla/example_mla_decode.py:230-265 (ref_program):
    query = [q, q_pe], key = [kv, k_pe] of one shared KV head, softmax(query key^T / sqrt(dv +
    dpe)) kv in fp32; also the TPU program tpu_demo/ppl/deepseek_mla/mla_decode.py:9-121 (same
    math with the natural-exp softmax and a singleton query axis). q [B, H, dv] or
    [B, H, 1, dv], q_pe likewise with dpe; kv [B, S, 1, dv], k_pe [B, S, 1, dpe]. Returns the
    shape of q in out_dtype (default q's dtype)."""
    shape = q.shape
    B, H = shape[0], shape[1]
    dv, dpe = q.shape[-1], q_pe.shape[-1]
    S = kv.shape[1]
    scale = (1.0 / math.sqrt(dv + dpe)) if sm_scale is None else sm_scale
    qq = torch.cat([q.reshape(B, H, dv).float(), q_pe.reshape(B, H, dpe).float()], dim=-1)
    kk = torch.cat([kv.reshape(B, S, dv).float(), k_pe.reshape(B, S, dpe).float()], dim=-1)
    vv = kv.reshape(B, S, dv).float()
    out = torch.empty(B, H, dv, dtype=torch.float32)
    for b in range(B):
        out[b] = torch.softmax((qq[b] @ kk[b].t()) * scale, dim=-1) @ vv[b]
    return out.reshape(shape).to(out_dtype or q.dtype)


# examples/deepseek_mla/torch_refs.py:6-78 (flash_split_ref + reduce_ref): split-KV partial
# outputs with log2-domain LSE, then the LSE-weighted combine. Restated over explicit splits of
# the token range (the kernel's partition, example_mla_decode_paged.py:140-144: blocks of
# block_N tokens, the first `total % num_split` splits take one extra block).
def mla_split_partition(seqlen: int, num_split: int, block_n: int):
    total = -(-seqlen // block_n)
    per, rem = divmod(total, num_split)
    bounds = []
    for s in range(num_split):
        nblk = per + (1 if s < rem else 0)
        start = (per * s + min(s, rem)) * block_n
        bounds.append((start, min(start + nblk * block_n, seqlen)))
    return bounds


def mla_split_combine_ref(q, q_pe, kv, k_pe, block_table, seqlens, page, sm_scale, num_split,
                          block_n=64, kv_scale=1.0, out_dtype=torch.bfloat16, store_dtype=None):
    """Split partials (flash_split_ref) and their LSE combine (reduce_ref). With store_dtype the
    partials are rounded to it before the combine, as the split program stores glse /
    Output_partial (example_mla_decode_paged.py:182-184) and its combine reads them back
    (:186-221); then returns (out, (glse [B, Hq, ns], partial [B, Hq, ns, dv])) as floats. A
    split without tokens has lse -inf and a zero partial."""
    B, Hq, dv = q.shape
    glse_all = torch.empty(B, Hq, num_split)
    part_all = torch.empty(B, Hq, num_split, dv)
    kv2 = kv.reshape(kv.shape[0], -1)
    kp2 = k_pe.reshape(k_pe.shape[0], -1)
    out = torch.zeros(B, Hq, dv, dtype=torch.float32)
    log2e = 1.0 / math.log(2.0)
    for b in range(B):
        L = int(seqlens[b])
        rows_all = paged_rows(block_table, L, b, page)
        rows = torch.arange(L)
        kvf = kv2[rows_all].float() * kv_scale
        kpf = kp2[rows_all].float() * kv_scale
        qb = torch.cat([q[b].float(), q_pe[b].float()], dim=1)
        parts, lses = [], []
        for (st, en) in mla_split_partition(L, num_split, block_n):
            if en <= st:
                parts.append(torch.zeros(Hq, dv))
                lses.append(torch.full((Hq,), float("-inf")))
                continue
            r = rows[st:en]
            s = (qb @ torch.cat([kvf[r], kpf[r]], 1).t()) * sm_scale * log2e  # log2 domain
            m = s.max(dim=-1).values
            p = torch.exp2(s - m[:, None])
            l = p.sum(-1)
            parts.append((p @ kvf[r]) / l[:, None])
            lses.append(torch.log2(l) + m)
        g = torch.stack(lses, -1)  # [Hq, ns]
        if store_dtype is not None:
            g = g.to(store_dtype).float()
            parts = [pt.to(store_dtype).float() for pt in parts]
        glse_all[b] = g
        part_all[b] = torch.stack(parts, 1)
        gmax = g.max(-1).values
        lse = torch.log2(torch.exp2(g - gmax[:, None]).sum(-1)) + gmax
        for i, part in enumerate(parts):
            out[b] += part * torch.exp2(g[:, i] - lse)[:, None]
    if store_dtype is not None:
        return out.to(out_dtype), (glse_all, part_all)
    return out.to(out_dtype)


# ------------------------------------------------------------------------------------------------
# FP8 e4m3fn (OCP) decode, numpy closed form: sign, 4-bit exponent (bias 7), 3-bit mantissa;
# exponent 0 is subnormal (m/8 * 2^-6); 0x7F / 0xFF are NaN; there is no infinity.
def fp8_e4m3fn_table() -> np.ndarray:
    t = np.empty(256, dtype=np.float32)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


def fp8_quantize(x: torch.Tensor):
    """Per-tensor e4m3 quantisation used by the MLA config: scale = amax / 448."""
    scale = float(x.abs().max()) / 448.0
    q = (x / scale).to(torch.float8_e4m3fn)
    return q, scale


def fp8_saturate_quantize(x: torch.Tensor, scale: float) -> torch.Tensor:
    """e4m3 codes of clamp(x / scale, -448, 448): fp32 division, then torch's RNE cast (the MLA
    config's cache construction, fp8_quantize above, for in-range values); NaN stays NaN."""
    return (x.float() / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)


def kv_append_fp8_ref(x: torch.Tensor, start, count, block_table, kv_bytes: np.ndarray,
                      page: int, scale: float) -> np.ndarray:
    """Paged KV append (the step before the MLA decode): token j < count[b] of sequence b goes to
    position p = start[b] + j, row block_table[b, p // page] * page + p % page
    (example_mla_decode_paged.py:62-63); positions beyond the table and rows outside the pool
    are skipped. Returns an updated copy of kv_bytes (uint8 [rows, D])."""
    out = kv_bytes.copy()
    codes = fp8_saturate_quantize(x, scale).view(torch.uint8).numpy()
    B, T = x.shape[0], x.shape[1]
    pages = block_table.shape[1]
    for b in range(B):
        for j in range(min(int(count[b]), T)):
            p = int(start[b]) + j
            if p < 0 or p >= pages * page:
                continue
            row = int(block_table[b, p // page]) * page + p % page
            if 0 <= row < out.shape[0]:
                out[row] = codes[b, j]
    return out


def paged_gather_ref(kv_bytes: np.ndarray, block_table: np.ndarray, seqlens: np.ndarray,
                     page: int) -> np.ndarray:
    """Concatenate every sequence's rows in token order (uint8 rows), numpy."""
    rows = []
    for b in range(block_table.shape[0]):
        j = np.arange(int(seqlens[b]))
        rows.append(block_table[b, j // page].astype(np.int64) * page + j % page)
    idx = np.concatenate(rows) if rows else np.zeros(0, np.int64)
    return kv_bytes[idx]
