"""GPU parity: MLA paged decode.

Oracle: restated run_torch_mla (examples/deepseek_mla/example_mla_decode_paged.py:259-308) with
an explicit block-table gather and fp8 dequantisation (decode(byte) * kv_scale).
Tolerances:
  * fp16 KV (the reference program as written): atol=rtol=1e-2 (:348);
  * FP8 KV (the config), stated separately and computed against the dequantised fp32
    reference: atol=2e-2, rtol=5e-2, and relative RMS error <= 3% (FP8_REL_RMS);
  * integer paths (block-table addressing, page gathers): bit-exact.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs, workloads
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


FP8_REL_RMS = 0.03
CONFIG_REL_RMS = 0.02
# share of elements allowed outside atol + rtol |ref| for FP8 KV: e4m3 P^T rounding at a few
# tokens per sequence (none at the config's lengths)
FP8_MISMATCH = 0.005


def _rel_rms(a, b):
    a, b = a.float(), b.float()
    return float(((a - b).pow(2).mean() / b.pow(2).mean()).sqrt())


def _run_fused(w, num_split, t=None):
    """Fused [rows, 576] fp8 cache and [B, Hq, 576] bf16 Q, through the C ABI."""
    a = w.attrs
    t = t or {k: v.to(DEV) for k, v in w.tensors.items()}
    q, kv = t["q"], t["kv"]
    out = torch.empty(a["B"], a["Hq"], a["dv"], dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.mla_workspace_bytes(a["B"], a["Hq"], a["dv"], num_split),
                     dtype=torch.uint8, device=DEV)
    ops.mla_decode(q[..., :512], q[..., 512:], kv[:, :512], kv[:, 512:], t["block_table"],
                   t["seqlens"], out, ws, a["page"], num_split, a["sm_scale"], t["kv_scale"])
    return out


def _oracle(w, seqs=None):
    a = w.attrs
    T = w.tensors
    seqs = list(range(a["B"])) if seqs is None else seqs
    q = T["q"][seqs]
    return ref.mla_decode_ref(q[..., :512], q[..., 512:], T["kv"][:, :512], T["kv"][:, 512:],
                              T["block_table"][seqs], T["seqlens"][seqs], a["page"],
                              a["sm_scale"], float(T["kv_scale"]))


def test_reference_program_fp16_split():
    """The reference's split program (fp16 Q and KV, glse/Output_partial params, out_idx=[8])."""
    B, Hq, dv, dpe, bs = 3, 128, 512, 64, 64
    max_seq = 512
    prog = programs.mla_decode(B, Hq, 1, max_seq, dv, dpe, 64, 64, 2, bs, dtype="float16")
    k = tilelang.compile(prog, out_idx=[8])
    assert k.plan.family == "mla" and k.plan.attrs["num_split"] == 2
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, Hq, dv + dpe, generator=g).half()
    kvp = torch.randn(B * max_seq, 1, dv + dpe, generator=g).half()
    bt = torch.arange(B * max_seq // bs, dtype=torch.int32).view(B, -1)
    sl = torch.tensor([511, 64, 200], dtype=torch.int32)
    glse = torch.empty(B, Hq, 2, dtype=torch.float16, device=DEV)
    opart = torch.empty(B, Hq, 2, dv, dtype=torch.float16, device=DEV)
    out = k(q[..., :dv].contiguous().to(DEV), q[..., dv:].contiguous().to(DEV),
            kvp[..., :dv].contiguous().to(DEV), kvp[..., dv:].contiguous().to(DEV),
            bt.to(DEV), sl.to(DEV), glse, opart)
    exp = ref.mla_decode_ref(q[..., :dv], q[..., dv:], kvp[..., :dv], kvp[..., dv:], bt, sl, bs,
                             1 / math.sqrt(dv + dpe), out_dtype=torch.float16)
    torch_assert_close(out.cpu(), exp, atol=1e-2, rtol=1e-2)
    # the split kernel's partials (:182-184), as the program stores them, and the combine of
    # the stored values (:186-221)
    comb, (g_ref, p_ref) = ref.mla_split_combine_ref(
        q[..., :dv], q[..., dv:], kvp[..., :dv], kvp[..., dv:], bt, sl, bs,
        1 / math.sqrt(dv + dpe), 2, block_n=64, out_dtype=torch.float16,
        store_dtype=torch.float16)
    torch_assert_close(glse.cpu().float(), g_ref, atol=2e-2, rtol=0)
    torch_assert_close(opart.cpu().float(), p_ref, atol=1e-2, rtol=1e-2)
    torch_assert_close(out.cpu(), comb, atol=1e-2, rtol=1e-2)


def test_split_program_partials_with_empty_splits():
    """Sequences with fewer 64-token blocks than splits (one block over 4 splits): the empty
    splits store lse -inf and zeros, and the output is the attention over the tokens."""
    B, Hq, dv, dpe, bs, ns = 2, 64, 512, 64, 64, 4
    prog = programs.mla_decode(B, Hq, 1, 256, dv, dpe, 64, 64, ns, bs, dtype="bfloat16")
    k = tilelang.compile(prog, out_idx=[8])
    g = torch.Generator().manual_seed(33)
    q = torch.randn(B, Hq, dv + dpe, generator=g).bfloat16()
    kvp = torch.randn(B * 256, 1, dv + dpe, generator=g).bfloat16()
    bt = torch.randperm(B * 4, generator=g).view(B, 4).to(torch.int32)
    sl = torch.tensor([40, 130], dtype=torch.int32)
    glse = torch.empty(B, Hq, ns, dtype=torch.bfloat16, device=DEV)
    opart = torch.empty(B, Hq, ns, dv, dtype=torch.bfloat16, device=DEV)
    out = k(q[..., :dv].contiguous().to(DEV), q[..., dv:].contiguous().to(DEV),
            kvp[..., :dv].contiguous().to(DEV), kvp[..., dv:].contiguous().to(DEV),
            bt.to(DEV), sl.to(DEV), glse, opart).cpu()
    comb, (g_ref, p_ref) = ref.mla_split_combine_ref(
        q[..., :dv], q[..., dv:], kvp[..., :dv], kvp[..., dv:], bt, sl, bs,
        1 / math.sqrt(dv + dpe), ns, block_n=64, out_dtype=torch.bfloat16,
        store_dtype=torch.bfloat16)
    assert torch.isinf(glse[0, :, 1:].float()).all() and not opart[0, :, 1:].any()
    torch_assert_close(glse.cpu().float(), g_ref, atol=0.13, rtol=0)
    torch_assert_close(opart.cpu().float(), p_ref, atol=2e-2, rtol=2e-2)
    torch_assert_close(out, comb, atol=2e-2, rtol=2e-2)
    exp = ref.mla_decode_ref(q[..., :dv], q[..., dv:], kvp[..., :dv], kvp[..., dv:], bt, sl, bs,
                             1 / math.sqrt(dv + dpe), out_dtype=torch.bfloat16)
    torch_assert_close(out, exp, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("ns", [4, 8])
def test_fp8_program_through_compile(ns):
    B, Hq, max_pages, page = 4, 128, 8, 64
    prog = programs.mla_decode(B, Hq, 1, max_pages * page, 512, 64, 64, 64, ns, page,
                               dtype="bfloat16", kv_dtype="float8_e4m3", out_dtype="bfloat16")
    k = tilelang.compile(prog, out_idx=[8])
    assert k.plan.attrs["kv_dtype"] == "float8_e4m3" and k.plan.attrs["kv_scale"] == 9
    w = workloads.mla(B=B, Hq=Hq, max_pages=max_pages, min_len=1, max_len=max_pages * page,
                      seed=32)
    T = w.tensors
    pool = T["kv"].view(B * max_pages * page, 1, 576)
    glse = torch.empty(B, Hq, ns, device=DEV)
    opart = torch.empty(B, Hq, ns, 512, device=DEV)
    out = k(T["q"][..., :512].contiguous().to(DEV), T["q"][..., 512:].contiguous().to(DEV),
            pool[..., :512].contiguous().to(DEV), pool[..., 512:].contiguous().to(DEV),
            T["block_table"].to(DEV), T["seqlens"].to(DEV), glse, opart,
            T["kv_scale"].to(DEV))
    # the program's own scale is 1/sqrt(576); the oracle follows the program
    exp = ref.mla_decode_ref(T["q"][..., :512], T["q"][..., 512:], T["kv"][:, :512],
                             T["kv"][:, 512:], T["block_table"], T["seqlens"], page,
                             1 / math.sqrt(576), float(T["kv_scale"]))
    torch_assert_close(out.cpu(), exp, atol=2e-2, rtol=5e-2)
    assert _rel_rms(out.cpu(), exp) < FP8_REL_RMS
    # the program's fp32 partials: each split's output (times kv_scale) and log2 sum-exp
    _, (g_ref, p_ref) = ref.mla_split_combine_ref(
        T["q"][..., :512], T["q"][..., 512:], T["kv"][:, :512], T["kv"][:, 512:],
        T["block_table"], T["seqlens"], page, 1 / math.sqrt(576), ns, block_n=64,
        kv_scale=float(T["kv_scale"]), store_dtype=torch.float32)
    _check_fp8_partials(glse.cpu(), opart.cpu(), g_ref, p_ref)


def _check_fp8_partials(glse, opart, g_ref, p_ref):
    """The fp8 path's (fp32) partials: a split's log2 sum-exp sums the e4m3-rounded P^T that
    weighs its output, so it follows the exact one within the rounding of P (at most 0.1 in
    log2 units, ~2% RMS in 2^lse); the split outputs within the FP8 output bounds."""
    live = torch.isfinite(g_ref)
    assert torch.equal(torch.isfinite(glse), live)
    d = (glse[live] - g_ref[live]).double()
    assert float(d.abs().max()) < 0.1, float(d.abs().max())
    assert float((torch.exp2(d) - 1).pow(2).mean().sqrt()) < 0.02
    torch_assert_close(opart, p_ref, atol=2e-2, rtol=5e-2, max_mismatched_ratio=FP8_MISMATCH)
    assert _rel_rms(opart, p_ref) < FP8_REL_RMS


def test_fp8_split_program_config():
    """The split program (example_mla_decode_paged.py, num_split 4, partials written) at the
    benchmark config: Output on every sequence, the partials on five."""
    w = workloads.mla()
    a = w.attrs
    B, Hq, page, mp = a["B"], a["Hq"], a["page"], a["max_pages"]
    prog = programs.mla_decode(B, Hq, 1, mp * page, 512, 64, 64, 64, 4, page,
                               dtype="bfloat16", kv_dtype="float8_e4m3", out_dtype="bfloat16")
    k = tilelang.compile(prog, out_idx=[8])
    T = w.tensors
    pool = T["kv"].view(B * mp * page, 1, 576)
    glse = torch.empty(B, Hq, 4, device=DEV)  # the fp8 program's partials are fp32
    opart = torch.empty(B, Hq, 4, 512, device=DEV)
    out = k(T["q"][..., :512].contiguous().to(DEV), T["q"][..., 512:].contiguous().to(DEV),
            pool[..., :512].contiguous().to(DEV), pool[..., 512:].contiguous().to(DEV),
            T["block_table"].to(DEV), T["seqlens"].to(DEV), glse, opart,
            T["kv_scale"].to(DEV)).cpu()
    sc = 1 / math.sqrt(576)
    exp = ref.mla_decode_ref(T["q"][..., :512], T["q"][..., 512:], T["kv"][:, :512],
                             T["kv"][:, 512:], T["block_table"], T["seqlens"], page, sc,
                             float(T["kv_scale"]))
    torch_assert_close(out, exp, atol=2e-2, rtol=5e-2)
    assert _rel_rms(out, exp) < CONFIG_REL_RMS
    sel = [0, 9, 31, 50, 63]
    _, (g_ref, p_ref) = ref.mla_split_combine_ref(
        T["q"][sel, :, :512], T["q"][sel, :, 512:], T["kv"][:, :512], T["kv"][:, 512:],
        T["block_table"][sel], T["seqlens"][sel], page, sc, 4, block_n=64,
        kv_scale=float(T["kv_scale"]), store_dtype=torch.float32)
    _check_fp8_partials(glse.cpu()[sel], opart.cpu()[sel], g_ref, p_ref)


@pytest.mark.parametrize("num_split", [1, 4, 8])
def test_fp8_config_full(num_split):
    """The benchmark config (B=64, Hq=128, L~U[1024,8192], page 64, random permutation table)."""
    w = workloads.mla()
    out = _run_fused(w, num_split).cpu()
    seqs = [0, 1, 17, 42, 63] if num_split != 4 else list(range(64))
    exp = _oracle(w, seqs)
    got = out[seqs]
    torch_assert_close(got, exp, atol=2e-2, rtol=5e-2)
    # the config itself runs at ~1.3-1.6% (one e4m3 term for P^T); 2% keeps a precision
    # regression from hiding under the 3% policy ceiling of the adversarial cases
    assert _rel_rms(got, exp) < CONFIG_REL_RMS


def test_split_invariance_and_page_permutation():
    """Output is (nearly) invariant to num_split, and exactly invariant to a joint permutation
    of the pool's pages and the block table (same values, same token order)."""
    w = workloads.mla(B=8, max_pages=16, min_len=1, max_len=1024, seed=33)
    t = {k: v.to(DEV) for k, v in w.tensors.items()}
    o1 = _run_fused(w, 1, t)
    o8 = _run_fused(w, 8, t)
    # P^T is rounded to e4m3 relative to each segment's running maximum, which depends on where
    # the splits cut the sequences: both results are within the FP8 tolerance of the oracle
    exp = _oracle(w)
    for o in (o1, o8):
        torch_assert_close(o.cpu(), exp, atol=2e-2, rtol=5e-2, max_mismatched_ratio=FP8_MISMATCH)
        assert _rel_rms(o.cpu(), exp) < FP8_REL_RMS
    n_pages = t["kv"].shape[0] // 64
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(34)).to(DEV)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(n_pages, device=DEV)
    kv_p = t["kv"].view(n_pages, 64, 576)[perm].reshape(-1, 576).contiguous()
    t2 = dict(t)
    t2["kv"] = kv_p
    t2["block_table"] = inv[t["block_table"].long()].to(torch.int32)
    o1p = _run_fused(w, 1, t2)
    assert torch.equal(o1, o1p)


def test_edge_lengths():
    """seqlen 1, exactly one page, a full table, and lengths not multiple of 32/64."""
    B, max_pages = 6, 4
    w = workloads.mla(B=B, max_pages=max_pages, min_len=1, max_len=256, seed=35)
    w.tensors["seqlens"] = torch.tensor([1, 64, 256, 33, 65, 255], dtype=torch.int32)
    out = _run_fused(w, 2).cpu()
    exp = _oracle(w)
    torch_assert_close(out, exp, atol=2e-2, rtol=5e-2, max_mismatched_ratio=FP8_MISMATCH)
    # seqlen 1: softmax over one token -> output is that token's latent row (dequantised)
    row = int(w.tensors["block_table"][0, 0]) * 64
    v0 = w.tensors["kv"][row, :512].float() * float(w.tensors["kv_scale"])
    torch_assert_close(out[0].float(), v0.expand(128, 512).to(torch.bfloat16).float(),
                       atol=1e-2, rtol=1e-2)


def test_fp8_decode_all_bytes():
    """Q = 0 makes the softmax uniform, so O = mean of the V rows: every non-NaN e4m3 byte
    value appears in V and is decoded exactly (OCP e4m3fn, bias 7)."""
    B, page, max_pages = 1, 64, 4
    L = 256
    vals = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)  # 254 codes
    rng = np.random.default_rng(36)
    kv_bytes = rng.choice(vals, size=(max_pages * page, 576)).astype(np.uint8)
    kv_bytes[:254, 0] = vals  # column 0 holds every code once
    kv = torch.from_numpy(kv_bytes).view(torch.float8_e4m3fn)
    bt = torch.arange(max_pages, dtype=torch.int32).view(1, -1)
    sl = torch.tensor([L], dtype=torch.int32)
    q = torch.zeros(B, 128, 576, dtype=torch.bfloat16)
    scale = torch.tensor([1.0 / 64], dtype=torch.float32)
    out = torch.empty(B, 128, 512, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(ops.mla_workspace_bytes(B, 128, 512, 1), dtype=torch.uint8, device=DEV)
    qd, kvd = q.to(DEV), kv.to(DEV)
    ops.mla_decode(qd[..., :512], qd[..., 512:], kvd[:, :512], kvd[:, 512:], bt.to(DEV),
                   sl.to(DEV), out, ws, page, 1, 0.1, scale.to(DEV))
    table = ref.fp8_e4m3fn_table()
    mean = torch.from_numpy(table[kv_bytes[:L, :512]].astype(np.float64).mean(0)) / 64
    got = out[0].cpu().double()
    assert torch.allclose(got, mean.expand(128, 512), atol=2e-3, rtol=8e-3)


def test_paged_gather_bit_exact():
    w = workloads.mla(B=16, max_pages=16, min_len=1, max_len=1024, seed=37)
    T = w.tensors
    sl = T["seqlens"]
    cu = torch.zeros(16, dtype=torch.int64)
    cu[1:] = torch.cumsum(sl.long(), 0)[:-1]
    total = int(sl.sum())
    kvb = T["kv"].view(torch.uint8)
    out = torch.empty(total, 576, dtype=torch.uint8, device=DEV)
    ops.paged_gather(kvb.to(DEV), T["block_table"].to(DEV), sl.to(DEV), cu.to(DEV), out, 64)
    exp = ref.paged_gather_ref(kvb.numpy(), T["block_table"].numpy(), sl.numpy(), 64)
    assert np.array_equal(out.cpu().numpy(), exp)


def test_out_of_pool_rows_read_as_zero():
    """A block table entry past the pool is not dereferenced (the row reads as zeros)."""
    T = workloads.mla(B=1, max_pages=2, min_len=128, max_len=128, seed=38).tensors
    bt = T["block_table"].clone()
    bt[0, 1] = 10_000  # page far outside the 2-page pool
    cu = torch.zeros(1, dtype=torch.int64)
    out = torch.full((128, 576), 7, dtype=torch.uint8, device=DEV)
    kvb = T["kv"].view(torch.uint8).to(DEV)
    ops.paged_gather(kvb, bt.to(DEV), T["seqlens"].to(DEV), cu.to(DEV), out, 64)
    assert int(out[64:].sum()) == 0
    assert torch.equal(out[:64].cpu(), T["kv"].view(torch.uint8)[int(bt[0, 0]) * 64:][:64])


def _split_program_cases(n, seed):
    import random
    r = random.Random(seed)
    return [(r.randint(1, 6), r.choice([128, 256]), r.choice([2, 3, 5, 8]), r.choice([64, 128]),
             r.choice([4, 8]), 200 + i) for i in range(n)]


@pytest.mark.parametrize("B,Hq,ns,page,mp,seed", _split_program_cases(6, seed=909))
def test_fp8_split_program_random(B, Hq, ns, page, mp, seed):
    """The split program on the segment path over random batches (lengths 0 .. the table's
    reach, several splits empty): partials and Output against the oracle."""
    print(f"split program B={B} Hq={Hq} ns={ns} page={page} pages={mp} seed={seed}", flush=True)
    w = workloads.mla(B=B, Hq=Hq, max_pages=mp, page=page, min_len=0, max_len=mp * page,
                      seed=seed)
    T = w.tensors
    prog = programs.mla_decode(B, Hq, 1, mp * page, 512, 64, 64, 64, ns, page,
                               dtype="bfloat16", kv_dtype="float8_e4m3", out_dtype="bfloat16")
    k = tilelang.compile(prog, out_idx=[8])
    pool = T["kv"].view(B * mp * page, 1, 576)
    glse = torch.full((B, Hq, ns), float("nan"), device=DEV)
    opart = torch.full((B, Hq, ns, 512), float("nan"), device=DEV)
    out = k(T["q"][..., :512].contiguous().to(DEV), T["q"][..., 512:].contiguous().to(DEV),
            pool[..., :512].contiguous().to(DEV), pool[..., 512:].contiguous().to(DEV),
            T["block_table"].to(DEV), T["seqlens"].to(DEV), glse, opart,
            T["kv_scale"].to(DEV)).cpu()
    sc = 1 / math.sqrt(576)
    _, (g_ref, p_ref) = ref.mla_split_combine_ref(
        T["q"][..., :512], T["q"][..., 512:], T["kv"][:, :512], T["kv"][:, 512:],
        T["block_table"], T["seqlens"], page, sc, ns, block_n=64,
        kv_scale=float(T["kv_scale"]), store_dtype=torch.float32)
    _check_fp8_partials(glse.cpu(), opart.cpu(), g_ref, p_ref)
    exp = ref.mla_decode_ref(T["q"][..., :512], T["q"][..., 512:], T["kv"][:, :512],
                             T["kv"][:, 512:], T["block_table"], T["seqlens"], page, sc,
                             float(T["kv_scale"]))
    live = T["seqlens"] > 0
    assert torch.equal(out[~live].float(), torch.zeros_like(out[~live].float()))
    if live.any():
        assert _rel_rms(out[live], exp[live]) < FP8_REL_RMS
