"""Pin the CPU oracle (oracle/ref.py, oracle/oracle.c) before trusting it.

The reference commits no golden vectors for this path (its demos only print allclose against
torch), so each oracle function is checked against something that does not restate its own
formula: an independent brute-force loop (pure Python / C fp64), a library routine that is a
special case (torch SDPA, numpy complex rotation, torch's float8 decode), and invariants a
plausible mistake would break (a dropped term, a transposed operand, a wrong sign or index).
"""
import ctypes
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import ROOT
from oracle import ref


def _liboracle():
    path = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
    if not os.path.exists(path):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(path)
    lib.oracle_fp8_e4m3fn_decode_one.restype = ctypes.c_float
    lib.oracle_paged_gather.restype = ctypes.c_int64
    return lib


# ---------------------------------------------------------------------------------------- RMSNorm
def test_rmsnorm_vs_c_fp64_brute_force():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 37, generator=g).half()
    w = (1 + 0.1 * torch.randn(37, generator=g)).half()
    lib = _liboracle()
    xf = np.ascontiguousarray(x.float().numpy())
    wf = np.ascontiguousarray(w.float().numpy())
    y = np.zeros((5, 37), dtype=np.float64)
    lib.oracle_rmsnorm_f64(xf.ctypes.data_as(ctypes.c_void_p), wf.ctypes.data_as(ctypes.c_void_p),
                           y.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(5),
                           ctypes.c_int64(37), ctypes.c_double(1e-6))
    got = ref.rmsnorm_ref(x, w, 1e-6).double().numpy()
    # one fp16 rounding of the fp64 value (half-ulp, relative 2^-11)
    assert np.all(np.abs(got - y) <= np.abs(y) * 2.0 ** -10 + 1e-7)


def test_rmsnorm_invariants():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(8, 4096, generator=g).half()
    y = ref.rmsnorm_ref(x, None, 1e-6).float()
    # unit RMS per row (w = 1)
    assert torch.allclose(y.pow(2).mean(-1).sqrt(), torch.ones(8), atol=2e-3)
    # scale invariance: rmsnorm(4x) == rmsnorm(x) (power-of-two scale is exact in fp16)
    assert torch.equal(ref.rmsnorm_ref((x.float() * 4).half(), None, 0.0),
                       ref.rmsnorm_ref(x, None, 0.0))
    # zero row stays zero with eps > 0
    assert torch.equal(ref.rmsnorm_ref(torch.zeros(1, 16).half(), None, 1e-6),
                       torch.zeros(1, 16).half())


# ------------------------------------------------------------------------------------------- GEMM
def test_matmul_vs_brute_force():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(3, 5, generator=g).half()
    b = torch.randn(5, 4, generator=g).half()
    exp = [[sum(float(a[i, k]) * float(b[k, j]) for k in range(5)) for j in range(4)]
           for i in range(3)]
    got = ref.matmul_ref(a, b, out_dtype=torch.float32)
    assert np.allclose(got.numpy(), np.array(exp), rtol=1e-6, atol=1e-6)
    # trans_b takes B as [N, K]
    got_t = ref.matmul_ref(a, b.t().contiguous(), out_dtype=torch.float32, trans_b=True)
    assert torch.equal(got, got_t)
    # non-square shapes catch a transposed operand
    a2 = torch.randn(2, 7, generator=g).half()
    b2 = torch.randn(7, 3, generator=g).half()
    assert ref.matmul_ref(a2, b2).shape == (2, 3)
    assert np.allclose(ref.matmul_ref(a2, b2, out_dtype=torch.float32).numpy(),
                       a2.double().numpy() @ b2.double().numpy(), atol=1e-5)


# ------------------------------------------------------------------------------------------- RoPE
def test_rope_tables_closed_form():
    cos, sin = ref.rope_cos_sin(300, 128, dtype=torch.float32)
    for pos, i in ((0, 0), (7, 3), (299, 63), (256, 1), (100, 10)):
        th = pos * 10000.0 ** (-2.0 * i / 128)
        assert abs(float(cos[pos, 2 * i]) - math.cos(th)) < 1e-5
        assert abs(float(sin[pos, 2 * i + 1]) - math.sin(th)) < 1e-5
    assert torch.equal(cos[:, 0::2], cos[:, 1::2]) and torch.equal(sin[:, 0::2], sin[:, 1::2])


def test_rope_vs_complex_rotation_and_invariants():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(50, 3, 64, generator=g)
    cos, sin = ref.rope_cos_sin(50, 64, dtype=torch.float32)
    out = ref.rope_ref(x, cos, sin).numpy()
    z = x.numpy()[..., 0::2] + 1j * x.numpy()[..., 1::2]
    th = np.arange(50)[:, None] * 10000.0 ** (-2.0 * np.arange(32) / 64)
    rot = z * np.exp(1j * th)[:, None, :]
    assert np.allclose(out[..., 0::2], rot.real, atol=1e-4)
    assert np.allclose(out[..., 1::2], rot.imag, atol=1e-4)
    # position 0 is the identity; pair norms are preserved
    assert np.allclose(out[0], x.numpy()[0], atol=0)
    assert np.allclose(np.abs(out[..., 0::2] + 1j * out[..., 1::2]), np.abs(z), atol=1e-4)


def test_rope_unpaired_tables_follow_rope_add():
    """Tables whose pairs differ: brute force over the program's tiles and the two strided adds
    of ppl_rope_add (codegen_ppl.cc:1809-1848), element by element in fp64."""
    g = torch.Generator().manual_seed(41)
    x, c, s = (torch.randn(3, 10, generator=g) for _ in range(3))
    out = ref.rope_ref(x, c, s).double().numpy()
    X, C, S = (t.double().numpy() for t in (x, c, s))
    for r in range(3):
        xc = [X[r, j] * C[r, j] for j in range(10)]
        xns = [(-X[r, j]) * S[r, j] for j in range(10)]
        xs = [X[r, j] * S[r, j] for j in range(10)]
        for i in range(5):
            assert abs(out[r, 2 * i] - (xc[2 * i] + xns[2 * i + 1])) < 1e-5
            assert abs(out[r, 2 * i + 1] - (xc[2 * i + 1] + xs[2 * i])) < 1e-5
    # and a wrong pairing (the even table entries for both outputs) differs
    alt = X[:, 0::2] * C[:, 0::2] - X[:, 1::2] * S[:, 0::2]
    assert np.abs(alt - out[:, 0::2]).max() > 1e-2


# ----------------------------------------------------------------------------------------- SwiGLU
def test_swiglu_vs_numpy_and_limits():
    g = torch.Generator().manual_seed(5)
    a = torch.randn(64, 33, generator=g).bfloat16()
    b = torch.randn(64, 33, generator=g).bfloat16()
    got = ref.swiglu_ref(a, b).double().numpy()
    an, bn = a.double().numpy(), b.double().numpy()
    exp = bn * an / (1.0 + np.exp(-an))
    assert np.all(np.abs(got - exp) <= np.abs(exp) * 2.0 ** -8 + 1e-30)
    z = torch.zeros(4).bfloat16()
    assert torch.equal(ref.swiglu_ref(z, torch.ones(4).bfloat16()), z)
    big = torch.full((2,), 30.0).bfloat16()
    assert torch.equal(ref.swiglu_ref(big, torch.ones(2).bfloat16()), big)


# --------------------------------------------------------------------------------- FlashAttention
@pytest.mark.parametrize("causal", [False, True])
def test_flashattn_vs_sdpa(causal):
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(2, 70, 3, 64, generator=g).bfloat16() for _ in range(3))
    got = ref.flashattn_ref(q, k, v, causal).float()
    exp = F.scaled_dot_product_attention(q.float().transpose(1, 2), k.float().transpose(1, 2),
                                         v.float().transpose(1, 2),
                                         is_causal=causal).transpose(1, 2)
    assert (got - exp).abs().max() < 1e-2


def test_flashattn_brute_force_and_invariants():
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, 3, 1, 2, generator=g) for _ in range(3))
    got = ref.flashattn_ref(q, k, v, causal=True, sm_scale=0.5)
    for i in range(3):
        s = [0.5 * sum(float(q[0, i, 0, d]) * float(k[0, j, 0, d]) for d in range(2))
             for j in range(i + 1)]
        m = max(s)
        p = [math.exp(x - m) for x in s]
        o = [sum(p[j] * float(v[0, j, 0, d]) for j in range(i + 1)) / sum(p) for d in range(2)]
        assert np.allclose(got[0, i, 0].numpy(), o, atol=1e-6)
    # causal first query attends to key 0 only -> V[0]; softmax rows sum to 1 (V = 1 -> O = 1)
    assert torch.allclose(got[0, 0], v[0, 0])
    ones = torch.ones(1, 5, 2, 8)
    assert torch.allclose(ref.flashattn_ref(torch.randn(1, 5, 2, 8), torch.randn(1, 5, 2, 8),
                                            ones, False), ones)


# -------------------------------------------------------------------------------------------- FP8
def test_fp8_table_vs_torch_and_c():
    t = ref.fp8_e4m3fn_table()
    torch_dec = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    lib = _liboracle()
    c_dec = np.array([lib.oracle_fp8_e4m3fn_decode_one(ctypes.c_uint8(b)) for b in range(256)],
                     dtype=np.float32)
    for arr in (torch_dec, c_dec):
        nan = np.isnan(t)
        assert np.array_equal(nan, np.isnan(arr))
        assert np.array_equal(t[~nan], arr[~nan])
    assert t[0x38] == 1.0 and t[0x7E] == 448.0 and t[0x01] == 2.0 ** -9 and t[0x08] == 2.0 ** -6
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF]) and t[0x80] == 0.0


def test_fp8_quantize_round_trip():
    x = torch.randn(1000, generator=torch.Generator().manual_seed(8))
    q8, scale = ref.fp8_quantize(x)
    assert abs(float(q8.float().abs().max()) - 448.0) < 1e-6
    rel = ((q8.float() * scale - x).abs() / x.abs().clamp_min(1e-3)).median()
    assert rel < 2 ** -4


# -------------------------------------------------------------------------------------------- MLA
def _mla_tiny(seed=9, B=2, Hq=3, dv=4, dpe=2, page=2, max_pages=3):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, dv, generator=g)
    qp = torch.randn(B, Hq, dpe, generator=g)
    n = B * max_pages * page
    kv = torch.randn(n, dv, generator=g)
    kp = torch.randn(n, dpe, generator=g)
    bt = torch.randperm(B * max_pages, generator=g).view(B, max_pages).to(torch.int32)
    sl = torch.tensor([5, 2], dtype=torch.int32)[:B]
    return q, qp, kv, kp, bt, sl


def test_mla_vs_token_loop():
    q, qp, kv, kp, bt, sl = _mla_tiny()
    got = ref.mla_decode_ref(q, qp, kv, kp, bt, sl, 2, 0.3, out_dtype=torch.float32)
    for b in range(2):
        for h in range(3):
            rows = [int(bt[b, j // 2]) * 2 + j % 2 for j in range(int(sl[b]))]
            s = [0.3 * (float(q[b, h] @ kv[r]) + float(qp[b, h] @ kp[r])) for r in rows]
            m = max(s)
            p = [math.exp(x - m) for x in s]
            o = sum(p[i] * kv[r].double() for i, r in enumerate(rows)) / sum(p)
            assert torch.allclose(got[b, h].double(), o, atol=1e-5)


def test_mla_identity_table_matches_reference_slicing():
    """With the reference's identity table (block_table = arange, begin = b * max_seqlen_pad),
    the gather reads exactly the contiguous slice run_torch_mla reads (:292-299)."""
    B, page, pages = 3, 4, 5
    bt = torch.arange(B * pages, dtype=torch.int32).view(B, pages)
    for b in range(B):
        rows = ref.paged_rows(bt, 13, b, page)
        assert torch.equal(rows, torch.arange(b * pages * page, b * pages * page + 13))


def test_mla_page_permutation_and_split_invariance():
    q, qp, kv, kp, bt, sl = _mla_tiny(seed=10)
    base = ref.mla_decode_ref(q, qp, kv, kp, bt, sl, 2, 0.7, out_dtype=torch.float32)
    perm = torch.randperm(6, generator=torch.Generator().manual_seed(11))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(6)
    kv2 = kv.view(6, 2, -1)[perm].reshape(12, -1)
    kp2 = kp.view(6, 2, -1)[perm].reshape(12, -1)
    bt2 = inv[bt.long()].to(torch.int32)
    assert torch.allclose(ref.mla_decode_ref(q, qp, kv2, kp2, bt2, sl, 2, 0.7,
                                             out_dtype=torch.float32), base, atol=1e-6)
    for ns in (1, 2, 3):
        sc = ref.mla_split_combine_ref(q, qp, kv, kp, bt, sl, 2, 0.7, ns, block_n=2,
                                       out_dtype=torch.float32)
        assert torch.allclose(sc, base, atol=1e-5)


def test_mla_split_partials_are_attention_over_each_split():
    """The stored partials of mla_split_combine_ref: split s's partial is the attention output
    over its own tokens and its glse the log2 sum-exp there (natural-log lse of mla_decode_ref
    over the same tokens, divided by ln 2); a split without tokens holds -inf and zeros."""
    g = torch.Generator().manual_seed(12)
    B, Hq, dv, dpe, page = 2, 3, 8, 4, 2
    q = torch.randn(B, Hq, dv, generator=g)
    qp = torch.randn(B, Hq, dpe, generator=g)
    kv = torch.randn(12, dv, generator=g)
    kp = torch.randn(12, dpe, generator=g)
    bt = torch.tensor([[3, 0, 5], [1, 4, 2]], dtype=torch.int32)
    sl = torch.tensor([5, 2], dtype=torch.int32)
    ns = 3
    out, (glse, part) = ref.mla_split_combine_ref(q, qp, kv, kp, bt, sl, page, 0.7, ns,
                                                  block_n=page, out_dtype=torch.float32,
                                                  store_dtype=torch.float32)
    assert torch.allclose(out, ref.mla_decode_ref(q, qp, kv, kp, bt, sl, page, 0.7,
                                                  out_dtype=torch.float32), atol=1e-5)
    for b in range(B):
        for s_, (st, en) in enumerate(ref.mla_split_partition(int(sl[b]), ns, page)):
            if en <= st:
                assert torch.isinf(glse[b, :, s_]).all() and not part[b, :, s_].any()
                continue
            sub_bt = bt[b:b + 1, st // page:]
            o, lse = ref.mla_decode_ref(q[b:b + 1], qp[b:b + 1], kv, kp, sub_bt,
                                        torch.tensor([en - st], dtype=torch.int32), page, 0.7,
                                        out_dtype=torch.float32, return_lse=True)
            assert torch.allclose(part[b, :, s_], o[0], atol=1e-5)
            assert torch.allclose(glse[b, :, s_], lse[0] / math.log(2.0), atol=1e-5)


def test_split_partition_rule():
    """example_mla_decode_paged.py:140-144: blocks dealt out, first (total % ns) get one more."""
    for L, ns, bn in ((4096, 4, 64), (65, 4, 64), (1, 8, 64), (1000, 3, 64)):
        parts = ref.mla_split_partition(L, ns, bn)
        covered = [t for st, en in parts for t in range(st, en)]
        assert covered == list(range(L))
        total = -(-L // bn)
        sizes = [-(-(en - st) // bn) if en > st else 0 for st, en in parts]
        assert sum(sizes) == total and max(sizes) - min(sizes) <= 1
        assert sizes == sorted(sizes, reverse=True)


def test_paged_gather_numpy_vs_c():
    rng = np.random.default_rng(12)
    B, page, pages = 4, 8, 6
    kv = rng.integers(0, 256, (B * pages * page, 24), dtype=np.uint8)
    bt = rng.permutation(B * pages).reshape(B, pages).astype(np.int32)
    sl = np.array([1, 48, 17, 0], dtype=np.int32)
    exp = ref.paged_gather_ref(kv, bt, sl, page)
    lib = _liboracle()
    out = np.zeros((int(sl.sum()), 24), dtype=np.uint8)
    n = lib.oracle_paged_gather(kv.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(24),
                                ctypes.c_int64(kv.shape[0]), bt.ctypes.data_as(ctypes.c_void_p),
                                sl.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(B),
                                ctypes.c_int64(pages), ctypes.c_int64(page),
                                out.ctypes.data_as(ctypes.c_void_p))
    assert n == sl.sum() and np.array_equal(out, exp)
    # the second sequence's 9th token lives in page bt[1, 1], slot 0
    off = 1 + 8
    assert np.array_equal(exp[off], kv[bt[1, 1] * page])


# ------------------------------------------------------------------------------- KV append (FP8)
def _e4m3_nearest_even(v: float, table: np.ndarray) -> int:
    """Brute force over the 256 codes: nearest finite e4m3 value to v, ties to the even
    mantissa (code with bit 0 clear), +0 for 0."""
    best, best_d = None, None
    for code in range(256):
        t = table[code]
        if np.isnan(t):
            continue
        d = abs(float(t) - v)
        if best is None or d < best_d or (d == best_d and (code & 1) == 0 and (best & 1) == 1):
            best, best_d = code, d
    if float(table[best]) == 0.0:
        best = 0x80 if math.copysign(1.0, v) < 0 and v != 0.0 else 0x00
    return best


def test_fp8_saturate_quantize_vs_brute_force_rne():
    """The quantiser (torch's RNE cast after clamping) picks the nearest e4m3 value with ties to
    even for every sample, including subnormals, exact ties and the +-448 saturation."""
    table = ref.fp8_e4m3fn_table()
    g = torch.Generator().manual_seed(31)
    finite = table[~np.isnan(table)].astype(np.float64)
    pos = np.unique(finite[finite > 0])
    mids = (pos[:-1] + pos[1:]) / 2.0  # exact ties between neighbours
    vals = torch.cat([torch.randn(400, generator=g) * 30, torch.rand(200, generator=g) * 0.004,
                      torch.tensor(mids, dtype=torch.float32), -torch.tensor(mids[:20], dtype=torch.float32),
                      torch.tensor([0.0, 447.9, 448.0, 460.0, 470.0, 1e6, -1e6, 2.0 ** -10,
                                    2.0 ** -10 + 2.0 ** -20])])
    codes = ref.fp8_saturate_quantize(vals, 1.0).view(torch.uint8).numpy()
    for v, c in zip(vals.tolist(), codes.tolist()):
        vs = min(max(v, -448.0), 448.0)
        assert c == _e4m3_nearest_even(vs, table), (v, hex(c))
    nan = ref.fp8_saturate_quantize(torch.tensor([float("nan")]), 1.0).float()
    assert torch.isnan(nan).all()


def test_kv_append_round_trip_through_gather():
    """Appending whole sequences into an empty pool and gathering them back through the block
    table (C-pinned gather) returns the quantised rows in token order."""
    g = torch.Generator().manual_seed(32)
    B, T, D, page, pages = 3, 20, 16, 4, 6
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    bt = torch.randperm(B * pages, generator=g).view(B, pages).to(torch.int32).numpy()
    count = np.array([20, 7, 0], dtype=np.int32)
    start = np.zeros(B, dtype=np.int32)
    pool = np.zeros((B * pages * page, D), dtype=np.uint8)
    scale = 0.01
    out = ref.kv_append_fp8_ref(x, start, count, bt, pool, page, scale)
    got = ref.paged_gather_ref(out, bt, count, page)
    q = ref.fp8_saturate_quantize(x, scale).view(torch.uint8).numpy()
    exp = np.concatenate([q[b, :count[b]] for b in range(B)])
    assert np.array_equal(got, exp)
    assert np.count_nonzero(out.any(axis=1)) <= int(count.sum())


def test_kv_append_incremental_equals_bulk_and_skips_out_of_range():
    g = torch.Generator().manual_seed(33)
    B, T, D, page, pages = 2, 9, 8, 4, 3
    x = torch.randn(B, T, D, generator=g).to(torch.float16)
    bt = np.array([[5, 0, 3], [1, 4, 2]], dtype=np.int32)
    pool = np.zeros((6 * page, D), dtype=np.uint8)
    bulk = ref.kv_append_fp8_ref(x, np.array([0, 2]), np.array([9, 7]), bt, pool, page, 0.05)
    step = pool
    for j in range(T):  # one token per call, decode-style
        xj = x[:, j:j + 1]
        cnt = np.array([1 if j < 9 else 0, 1 if j < 7 else 0])
        step = ref.kv_append_fp8_ref(xj, np.array([j, 2 + j]), cnt, bt, step, page, 0.05)
    assert np.array_equal(bulk, step)
    # positions past the table (3 pages * 4 = 12) and rows outside the pool are skipped
    out = ref.kv_append_fp8_ref(x, np.array([10, 0]), np.array([9, 1]), np.array(
        [[5, 0, 3], [99, 4, 2]], dtype=np.int32), pool, page, 0.05)
    assert np.count_nonzero(out.any(axis=1)) == 2  # positions 10, 11 of sequence 0 only


def test_flashattn_gqa_equals_mha_on_repeated_kv():
    """Grouped K/V heads: the oracle equals the MHA oracle on K/V repeated per group
    (example_gqa_fwd_bshd.py:195-196, repeat_interleave), for causal and full attention."""
    g = torch.Generator().manual_seed(31)
    B, S, H, Hkv, D = 2, 20, 6, 2, 8
    q = torch.randn(B, S, H, D, generator=g)
    k = torch.randn(B, S, Hkv, D, generator=g)
    v = torch.randn(B, S, Hkv, D, generator=g)
    for causal in (False, True):
        got = ref.flashattn_ref(q, k, v, causal)
        exp = ref.flashattn_ref(q, k.repeat_interleave(H // Hkv, dim=2),
                                v.repeat_interleave(H // Hkv, dim=2), causal)
        assert torch.equal(got, exp)
        # and heads of one group differ from the next group's (the mapping is h // G, not h % H_kv)
        assert not torch.allclose(got[:, :, 0], got[:, :, H // Hkv])


@pytest.mark.parametrize("dt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_gemm_fp8_ref_against_fp64_brute_force(dt):
    """fp8 GEMM oracle: exact fp8 decode and fp32 accumulation against an fp64 triple loop of the
    decoded values (products of fp8 values are exact; a 48-term sum stays within fp32 rounding),
    and the fp8 output equals torch's RNE cast of that fp64 result except at rounding ties."""
    g = torch.Generator().manual_seed(32)
    a = (torch.randn(5, 48, generator=g) * 3).to(dt)
    b = (torch.randn(7, 48, generator=g) * 3).to(dt)
    got = ref.gemm_fp8_ref(a, b)
    A, Bm = a.double().numpy(), b.double().numpy()
    exp = np.zeros((5, 7))
    for i in range(5):
        for j in range(7):
            exp[i, j] = sum(A[i, k] * Bm[j, k] for k in range(48))
    assert np.allclose(got.double().numpy(), exp, rtol=1e-6, atol=1e-5)
    q = ref.gemm_fp8_ref(a, b, out_dtype=dt).float().numpy()
    e8 = torch.from_numpy(exp).float().to(dt).float().numpy()
    assert (q == e8).mean() > 0.97


def test_sigmoid_ref_closed_form():
    """sigmoid against the fp64 closed form 1 / (1 + e^-x), its symmetry and s(0) = 1/2."""
    x = torch.linspace(-30, 30, 2001)
    exp = 1.0 / (1.0 + np.exp(-x.double().numpy()))
    assert np.allclose(ref.sigmoid_ref(x).double().numpy(), exp, rtol=1e-6, atol=1e-7)
    assert float(ref.sigmoid_ref(torch.zeros(1))[0]) == 0.5
    assert torch.allclose(ref.sigmoid_ref(-x), 1 - ref.sigmoid_ref(x), atol=1e-6)


def test_gather_ref_against_loop():
    g = torch.Generator().manual_seed(33)
    param = torch.randn(10, 5, generator=g)
    index = torch.tensor([[3], [0], [9], [10], [-1], [3]], dtype=torch.int32)  # 10, -1: out of range
    got = ref.gather_ref(param, index)
    for i, v in enumerate(index.view(-1).tolist()):
        u = v & 0xFFFFFFFF
        exp = param[u] if u < 10 else torch.zeros(5)
        assert torch.equal(got[i], exp)


@pytest.mark.parametrize("descending", [True, False])
def test_topk_ref_against_python_sort(descending):
    """Full stable order with ties, NaN (above every number) and -0.0 == +0.0, checked against
    Python's sorted() with an explicit (value class, value, index) key."""
    vals = [1.5, -0.0, float("nan"), 0.0, 2.0, 1.5, float("-inf"), float("inf"), -3.0, 0.0,
            float("nan"), 1.5]
    src = torch.tensor(vals, dtype=torch.float32)
    got_v, got_i = ref.topk_ref(src, descending)

    def key(i):
        v = vals[i]
        cls = 1 if math.isnan(v) else 0
        val = 0.0 if math.isnan(v) else v
        return (-cls, -val, i) if descending else (cls, val, i)

    order = sorted(range(len(vals)), key=key)
    assert got_i.tolist() == order
    assert torch.equal(got_v.view(torch.int32), src[order].view(torch.int32))
    u = torch.tensor([5, 0, 4294967295, 7, 5], dtype=torch.int64).to(torch.uint32)
    uv, ui = ref.topk_ref(u, descending)
    uorder = sorted(range(5), key=lambda i: ((-1 if descending else 1) * [5, 0, 4294967295, 7, 5][i], i))
    assert ui.tolist() == uorder


def test_row_reduce_ref():
    x = torch.tensor([[1.0, -2.0, 3.5], [float("nan"), 1.0, 2.0]])
    assert ref.row_reduce_ref(x, "max").view(-1)[0] == 3.5
    assert torch.isnan(ref.row_reduce_ref(x, "max").view(-1)[1])
    assert ref.row_reduce_ref(x, "sum").view(-1)[0] == 2.5


def _varlen_case(lens_q, lens_k, H, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    cu_q = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), H, D, generator=g)
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g)
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g)
    return q, k, v, cu_q, cu_k


def test_flashattn_varlen_equal_lengths_is_the_dense_oracle():
    """All sequences of one length: the unpadded layout is BSHD flattened, so the varlen oracle
    equals flashattn_ref (itself pinned by SDPA), causal and not."""
    B, S, H, D = 3, 17, 4, 8
    q, k, v, cu_q, cu_k = _varlen_case([S] * B, [S] * B, H, H, D, seed=40)
    for causal in (False, True):
        got = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal)
        exp = ref.flashattn_ref(q.view(B, S, H, D), k.view(B, S, H, D), v.view(B, S, H, D),
                                causal).float()
        torch.testing.assert_close(got.view(B, S, H, D), exp, rtol=1e-6, atol=1e-6)


def test_flashattn_varlen_matches_padded_sdpa():
    """The example's own construction (example_mha_fwd_varlen.py:385-426): pad each sequence to
    the longest, mask padded keys, run attention on the padded batch, unpad. Here the padded
    attention is torch's SDPA with a boolean key mask."""
    lens_q, lens_k, H, Hkv, D = [5, 1, 13, 9], [7, 4, 13, 2], 4, 2, 16
    q, k, v, cu_q, cu_k = _varlen_case(lens_q, lens_k, H, Hkv, D, seed=41)
    got = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k)
    Sq, Sk, B = max(lens_q), max(lens_k), len(lens_q)
    qp = torch.zeros(B, H, Sq, D)
    kp = torch.zeros(B, H, Sk, D)
    vp = torch.zeros(B, H, Sk, D)
    keep = torch.zeros(B, 1, 1, Sk, dtype=torch.bool)
    for b in range(B):
        qs = q[cu_q[b]:cu_q[b + 1]]
        ks = k[cu_k[b]:cu_k[b + 1]].repeat_interleave(H // Hkv, dim=1)
        vs = v[cu_k[b]:cu_k[b + 1]].repeat_interleave(H // Hkv, dim=1)
        qp[b, :, :lens_q[b]] = qs.transpose(0, 1)
        kp[b, :, :lens_k[b]] = ks.transpose(0, 1)
        vp[b, :, :lens_k[b]] = vs.transpose(0, 1)
        keep[b, ..., :lens_k[b]] = True
    op = F.scaled_dot_product_attention(qp, kp, vp, attn_mask=keep)
    for b in range(B):
        exp = op[b, :, :lens_q[b]].transpose(0, 1)
        torch.testing.assert_close(got[cu_q[b]:cu_q[b + 1]], exp, rtol=1e-5, atol=1e-5)


def test_flashattn_varlen_causal_alignment_and_edges():
    """Causal keeps key j <= i + nk - nq (bottom-right): a one-query sequence sees every key (a
    top-left mask would let it see key 0 only) and equal lengths give SDPA's is_causal. A
    sequence without keys gives zero rows; rows at positions >= max_seqlen_q stay unwritten."""
    H, D = 2, 8
    q, k, v, cu_q, cu_k = _varlen_case([1, 6, 4, 3], [9, 6, 0, 5], H, H, D, seed=42)
    full = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal=False)
    causal = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal=True)
    torch.testing.assert_close(causal[0], full[0])  # nq = 1: all 9 keys visible
    qs, ks, vs = (t.transpose(0, 1) for t in (q[1:7], k[9:15], v[9:15]))
    exp = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True).transpose(0, 1)
    torch.testing.assert_close(causal[1:7], exp, rtol=1e-5, atol=1e-5)
    assert torch.equal(full[7:11], torch.zeros(4, H, D))  # nk = 0
    # nq = 3 over nk = 5: query 0 sees keys 0..2 only, query 2 all five
    s0 = (q[11, 0] @ k[15:20, 0].t()) / math.sqrt(D)
    p0 = torch.softmax(s0[:3], dim=0)
    torch.testing.assert_close(causal[11, 0], p0 @ v[15:18, 0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(causal[13], full[13])
    cut = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, max_seqlen_q=4)
    assert torch.isnan(cut[5:7]).all() and torch.equal(cut[1:5], full[1:5])


def test_flashattn_varlen_gqa_equals_repeated_kv():
    lens = [3, 8, 5]
    q, k, v, cu_q, cu_k = _varlen_case(lens, lens, 6, 2, 8, seed=43)
    for causal in (False, True):
        got = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal)
        exp = ref.flashattn_varlen_ref(q, k.repeat_interleave(3, dim=1),
                                       v.repeat_interleave(3, dim=1), cu_q, cu_k, causal)
        assert torch.equal(got, exp)


def test_flashattn_bhsd_matches_sdpa_and_the_other_layouts():
    """Head-major oracle: equal lengths give SDPA (its is_causal is the top-left tril, equal to
    the bottom-right mask at S_q == S_kv) and the BSHD oracle on transposed tensors; unequal
    lengths give the variable-length oracle with one sequence per batch (its bottom-right causal
    mask and zero rows are pinned above); grouped K/V heads equal repeated ones."""
    g = torch.Generator().manual_seed(44)
    B, H, S, D = 2, 3, 9, 8
    q, k, v = (torch.randn(B, H, S, D, generator=g) for _ in range(3))
    for causal in (False, True):
        got = ref.flashattn_bhsd_ref(q, k, v, causal)
        exp = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-5)
        bshd = ref.flashattn_ref(*(t.transpose(1, 2) for t in (q, k, v)), causal)
        torch.testing.assert_close(got, bshd.transpose(1, 2), rtol=1e-6, atol=1e-6)
    Hkv = 1
    for Sq, Sk in ((5, 12), (12, 5), (7, 0)):
        q = torch.randn(B, H, Sq, D, generator=g)
        k, v = (torch.randn(B, Hkv, Sk, D, generator=g) for _ in range(2))
        cu_q = torch.arange(B + 1, dtype=torch.int32) * Sq
        cu_k = torch.arange(B + 1, dtype=torch.int32) * Sk
        for causal in (False, True):
            got = ref.flashattn_bhsd_ref(q, k, v, causal)
            exp = ref.flashattn_varlen_ref(q.permute(0, 2, 1, 3).reshape(B * Sq, H, D),
                                           k.permute(0, 2, 1, 3).reshape(B * Sk, Hkv, D),
                                           v.permute(0, 2, 1, 3).reshape(B * Sk, Hkv, D),
                                           cu_q, cu_k, causal)
            torch.testing.assert_close(got, exp.view(B, Sq, H, D).permute(0, 2, 1, 3),
                                       rtol=1e-6, atol=1e-6)
            rep = ref.flashattn_bhsd_ref(q, k.repeat_interleave(H, 1), v.repeat_interleave(H, 1),
                                         causal)
            assert torch.equal(got, rep)
    # S_q > S_kv causal: the first S_q - S_kv queries see no key and get zeros
    got = ref.flashattn_bhsd_ref(*(torch.randn(1, 1, s, 4, generator=g) for s in (6, 2, 2)), True)
    assert torch.equal(got[0, 0, :4], torch.zeros(4, 4)) and got[0, 0, 4:].abs().sum() > 0


def test_flashattn_rows_ref_equals_full_oracle_rows():
    """The row-subset oracle is the full oracle's rows (causal and not, grouped K/V heads)."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 96, 4, 32, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 96, 2, 32, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 96, 2, 32, generator=g).to(torch.bfloat16)
    rows = [0, 1, 17, 50, 95]
    for causal in (True, False):
        full = ref.flashattn_ref(q, k, v, causal).float()
        sub = ref.flashattn_rows_ref(q, k, v, causal, rows)
        assert torch.allclose(sub.to(torch.bfloat16).float(), full[:, rows], atol=1e-2,
                              rtol=1e-2)
        # first causal query sees only key 0: its output is V[0] of its K/V head
        if causal:
            assert torch.allclose(sub[:, 0], v[:, 0].float().repeat_interleave(2, dim=1),
                                  atol=1e-6)


def test_mla_nopage_ref_is_the_paged_oracle_on_an_identity_table():
    """Non-paged MLA (example_mla_decode.py ref_program) equals the paged oracle when the cache
    is laid out sequence by sequence (one page of S tokens per sequence, table row b = [b]),
    for the upstream [B, H, d] and the TPU demo's [B, H, 1, d] query layouts; a one-token cache
    returns its latent row."""
    g = torch.Generator().manual_seed(11)
    B, H, S, dv, dpe = 3, 8, 40, 32, 4
    q = torch.randn(B, H, dv, generator=g).half()
    qpe = torch.randn(B, H, dpe, generator=g).half()
    kv = torch.randn(B, S, 1, dv, generator=g).half()
    kpe = torch.randn(B, S, 1, dpe, generator=g).half()
    got = ref.mla_decode_nopage_ref(q, qpe, kv, kpe).float()
    bt = torch.arange(B, dtype=torch.int32).view(B, 1)
    sl = torch.full((B,), S, dtype=torch.int32)
    exp = ref.mla_decode_ref(q, qpe, kv.reshape(B * S, dv), kpe.reshape(B * S, dpe), bt, sl, S,
                             1 / math.sqrt(dv + dpe), out_dtype=torch.float32)
    assert torch.allclose(got, exp, atol=2e-3, rtol=2e-3)
    got4 = ref.mla_decode_nopage_ref(q.unsqueeze(2), qpe.unsqueeze(2), kv, kpe)
    assert got4.shape == (B, H, 1, dv)
    assert torch.equal(got4.squeeze(2), ref.mla_decode_nopage_ref(q, qpe, kv, kpe))
    one = ref.mla_decode_nopage_ref(q, qpe, kv[:, :1], kpe[:, :1]).float()
    assert torch.allclose(one, kv[:, 0].float().expand(B, H, dv), atol=1e-3)


def test_elementwise_program_refs_against_float64_numpy():
    """exp / row-broadcast product / scale-shift / add oracles against float64 numpy (and the
    closed forms e^0 = 1, e^1 = e), with fp32 rounding as the only difference."""
    g = torch.Generator().manual_seed(12)
    a = torch.randn(7, 5, generator=g)
    b = torch.randn(7, 1, generator=g)
    c = torch.randn(7, 5, generator=g)
    an, bn, cn = (x.double().numpy() for x in (a, b, c))
    assert np.allclose(ref.ppl_exp_ref(a).numpy(), np.exp(an), rtol=2e-7)
    assert float(ref.ppl_exp_ref(torch.tensor([0.0]))) == 1.0
    assert abs(float(ref.ppl_exp_ref(torch.tensor([1.0]))) - math.e) < 3e-7
    assert np.allclose(ref.ppl_mul_rows_ref(a, b).numpy(), an * bn, rtol=2e-7)
    assert np.allclose(ref.ppl_scale_shift_ref(a, 1 / 8192, 1e-12).numpy(), an / 8192 + 1e-12,
                       rtol=2e-7, atol=1e-18)
    assert np.allclose(ref.ppl_add_ref(a, c).numpy(), an + cn, rtol=2e-7)
    # bf16 tiles: the product is rounded before the shift is added
    ab = a.to(torch.bfloat16)
    t = (ab.double() / 8192).to(torch.bfloat16).double() + 1e-12
    assert torch.equal(ref.ppl_scale_shift_ref(ab, 1 / 8192, 1e-12), t.to(torch.bfloat16))


def test_mha_inference_ref_and_split_combine():
    """Split-KV inference oracle: the full-softmax reference equals SDPA on the head-major view
    (S_q != S_kv, non-causal); the restated split + combine algorithm of the program, with fp32
    intermediates, equals it to fp32 rounding for any split count, and with the program's fp16
    glse / Output_partial to fp16 rounding. A plausible slip (a split weight without the lse
    offset, a dropped alpha rescale, a missing scale) breaks one of these."""
    g = torch.Generator().manual_seed(45)
    B, Sq, Skv, H, D = 2, 5, 64, 3, 16
    q = torch.randn(B, Sq, H, D, generator=g).half()
    k = torch.randn(B, Skv, H, D, generator=g).half()
    v = torch.randn(B, Skv, H, D, generator=g).half()
    full = ref.mha_inference_ref(q, k, v)
    sdpa = F.scaled_dot_product_attention(*(t.float().transpose(1, 2) for t in (q, k, v)))
    torch.testing.assert_close(full, sdpa.transpose(1, 2), rtol=1e-5, atol=1e-5)
    for ns, bn in ((1, 64), (2, 16), (4, 8), (8, 8)):
        got, (glse, part) = ref.mha_split_combine_ref(q, k, v, ns, bn, store_dtype=torch.float32)
        # P rounded to fp16 before P V (the program's acc_s_cast): ~1e-3 of the output
        torch.testing.assert_close(got, full, rtol=2e-3, atol=2e-3)
        assert glse.shape == (B, H, ns, Sq) and part.shape == (B, Sq, H, ns, D)
        got16, _ = ref.mha_split_combine_ref(q, k, v, ns, bn)
        torch.testing.assert_close(got16, full, rtol=5e-3, atol=5e-3)
    # one split: its stored output is the attention output, its lse the log2 sum-exp
    got, (glse, part) = ref.mha_split_combine_ref(q, k, v, 1, 64, store_dtype=torch.float32)
    s = torch.einsum("bqhd,bkhd->bhqk", q.float(), k.float()) / math.sqrt(D)
    torch.testing.assert_close(glse[:, :, 0], torch.logsumexp(s, -1) / math.log(2), rtol=1e-5,
                               atol=1e-5)


def test_mlp_ref_composition_and_loops():
    """MLP oracle: equals the pinned gemm / SwiGLU oracles composed (matmul_ref with trans_b,
    swiglu_ref), and a scalar-loop evaluation of the program's steps on a tiny case (gate/up
    rounded to bf16, SiLU(g) = g / (1 + e^-g) in fp32, one rounding of the product)."""
    g = torch.Generator().manual_seed(46)
    M, Hd, I = 6, 8, 12
    x = torch.randn(M, Hd, generator=g).bfloat16()
    wg, wu = (torch.randn(I, Hd, generator=g).bfloat16() for _ in range(2))
    wd = torch.randn(Hd, I, generator=g).bfloat16()
    got = ref.mlp_ref(x, wg, wu, wd)
    gate = ref.matmul_ref(x, wg, torch.bfloat16, trans_b=True)
    up = ref.matmul_ref(x, wu, torch.bfloat16, trans_b=True)
    exp = ref.matmul_ref(ref.swiglu_ref(gate, up), wd, torch.bfloat16, trans_b=True)
    torch.testing.assert_close(got.float(), exp.float(), rtol=0, atol=0)
    xf, wgf, wuf, wdf = (t.float().tolist() for t in (x, wg, wu, wd))
    for r in range(M):
        h = []
        for i in range(I):
            gv = float(torch.tensor(sum(xf[r][k] * wgf[i][k] for k in range(Hd))).bfloat16())
            uv = float(torch.tensor(sum(xf[r][k] * wuf[i][k] for k in range(Hd))).bfloat16())
            h.append(float(torch.tensor(gv / (1.0 + math.exp(-gv)) * uv).bfloat16()))
        for c in range(Hd):
            o = float(torch.tensor(sum(h[i] * wdf[c][i] for i in range(I))).bfloat16())
            assert abs(o - float(got[r, c])) <= 2 ** -7 * abs(o) + 1e-6
    # the all-fp32 program (mlp_fp32.py): fp32 tiles rounded to bf16 before the gemms (RNE,
    # torch's cast), the bf16 result widened exactly: the bf16 oracle on the rounded inputs
    x32 = x.float() + torch.randn(M, Hd, generator=g) * 1e-3
    got32 = ref.mlp_ref(x32, wg.float(), wu.float(), wd.float(), operand_dtype=torch.bfloat16)
    assert got32.dtype == torch.float32
    assert torch.equal(got32, ref.mlp_ref(x32.bfloat16(), wg, wu, wd).float())
