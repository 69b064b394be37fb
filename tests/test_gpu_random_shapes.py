"""GPU parity over seeded random shapes for the tiled MFMA kernels (16x16 operand layouts, LDS
swizzles, edge masking): GEMM (both B layouts, fp16 / bf16, ragged M, N, K, skinny M <= 16), FP8 GEMM and
FlashAttention (causal or not, grouped K/V heads, head dim 64 and 128, ragged S), and the other
attention layouts over random shapes and head dims 8-256: head-major with independent query and
key lengths, variable length, split-KV inference with its partials. Each case prints its shape
before it runs. Tolerances follow the family tests: GEMM 1e-2 (the demo's),
FP8 GEMM fp32 output 1e-4 relative + 1e-2 absolute (summation order), FA 2e-2 (P is rounded to
the input type before P V).
"""
import math
import random

import pytest
import torch

from tilelang.jit.adapter.mi355x import ops
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gemm_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        M = r.choice([17, 100, 255, 256, 257, 513, 700])
        N = r.choice([8, 64, 200, 256, 264, 520, 1000])
        K = 8 * r.randint(1, 140)
        out.append((M, N, K, r.random() < 0.5, r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("M,N,K,trans_b,dt", _gemm_cases(16, seed=2024))
def test_gemm_random(M, N, K, trans_b, dt):
    print(f"gemm M={M} N={N} K={K} trans_b={trans_b} {dt}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N * 13 + K)
    a = (torch.rand(M, K, generator=g) * 2 - 1).to(dt)
    b = (torch.rand(N, K, generator=g) * 2 - 1).to(dt) if trans_b else \
        (torch.rand(K, N, generator=g) * 2 - 1).to(dt)
    c = torch.empty(M, N, dtype=dt, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c, trans_b=trans_b)
    torch_assert_close(c.cpu().float(), ref.matmul_ref(a, b, torch.float32, trans_b),
                       atol=1e-2, rtol=1e-2)


def _skinny_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        M = r.randint(1, 16)
        N = 8 * r.randint(1, 300)
        K = r.choice([8 * r.randint(1, 64), 32 * r.randint(1, 128), 8 * r.randint(500, 700)])
        out.append((M, N, K, r.random() < 0.25, r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("M,N,K,trans_b,dt", _skinny_cases(16, seed=77))
def test_gemm_skinny_random(M, N, K, trans_b, dt):
    """M <= 16 takes the skinny kernels: A staged in LDS for row-major B and K <= 4096, A read
    per block otherwise (K past 4096, B^T); ragged N and K not a multiple of 32 included."""
    test_gemm_random(M, N, K, trans_b, dt)


@pytest.mark.parametrize("M,N,K", [(300, 520, 640), (256, 256, 128), (1000, 264, 2048),
                                   (17, 1000, 384)])
def test_gemm_fp8_random(M, N, K):
    print(f"gemm_fp8 M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(torch.float8_e4m3fn)
    b = torch.randn(N, K, generator=g).to(torch.float8_e4m3fn)
    c = torch.empty(M, N, dtype=torch.float32, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c, trans_b=True)
    torch.testing.assert_close(c.cpu(), ref.gemm_fp8_ref(a, b), rtol=1e-4, atol=1e-2)


def _fa_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        D = r.choice([64, 128])
        Hkv = r.choice([1, 2, 4])
        H = Hkv * r.choice([1, 2, 3])
        out.append((r.randint(1, 2), r.choice([1, 65, 200, 256, 300, 513, 777]), H, Hkv, D,
                    r.random() < 0.5, r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("B,S,H,Hkv,D,causal,dt", _fa_cases(12, seed=77))
def test_flashattn_random(B, S, H, Hkv, D, causal, dt):
    print(f"flashattn B={B} S={S} H={H} Hkv={Hkv} D={D} causal={causal} {dt}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + S + H + D)
    q = torch.randn(B, S, H, D, generator=g).to(dt)
    k = torch.randn(B, S, Hkv, D, generator=g).to(dt)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dt)
    o = torch.empty_like(q, device=DEV)
    sc = 1 / math.sqrt(D)
    ops.flash_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, causal, sc)
    exp = ref.flashattn_ref(q.float(), k.float(), v.float(), causal, sc)
    torch_assert_close(o.cpu().float(), exp, atol=2e-2, rtol=2e-2)


def _layout_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        D = r.choice([8, 24, 64, 72, 128, 136, 256])
        Hkv = r.choice([1, 2])
        out.append((r.randint(1, 2), r.choice([1, 17, 128, 200, 333]),
                    r.choice([1, 63, 300, 512, 1000]), Hkv * r.choice([1, 3]), Hkv, D,
                    r.random() < 0.5, r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,D,causal,dt", _layout_cases(8, seed=91))
def test_flashattn_bhsd_random(B, Sq, Sk, H, Hkv, D, causal, dt):
    """Head-major attention with independent query and key lengths (bottom-right causal mask;
    a query that sees no key gets zeros), tiled and per-query head dims."""
    print(f"bhsd B={B} Sq={Sq} Sk={Sk} H={H} Hkv={Hkv} D={D} causal={causal} {dt}", flush=True)
    g = torch.Generator().manual_seed(B * 7919 + Sq * 31 + Sk + D)
    q = torch.randn(B, H, Sq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Sk, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Sk, D, generator=g).to(dt)
    o = torch.full((B, H, Sq, D), float("nan"), dtype=dt, device=DEV)
    sc = 1 / math.sqrt(D)
    ops.flash_attn_bhsd_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, causal, sc)
    torch_assert_close(o.cpu().float(), ref.flashattn_bhsd_ref(q, k, v, causal, sc),
                       atol=2e-2, rtol=2e-2)


def _varlen_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        B = r.randint(1, 5)
        lq = [r.choice([0, 1, 50, 128, 257, 600]) for _ in range(B)]
        lq[0] = max(lq[0], 1)
        causal = r.random() < 0.4
        lk = [x + r.choice([0, 64, 100]) if causal else r.choice([x, 1, 300, 700]) for x in lq]
        Hkv = r.choice([1, 2])
        out.append((lq, lk, Hkv * r.choice([1, 2]), Hkv, r.choice([32, 64, 128]), causal,
                    r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("lq,lk,H,Hkv,D,causal,dt", _varlen_cases(8, seed=92))
def test_flashattn_varlen_random(lq, lk, H, Hkv, D, causal, dt):
    """Unpadded sequences of ragged lengths (empty ones included) through cu_seqlens."""
    print(f"varlen lq={lq} lk={lk} H={H} Hkv={Hkv} D={D} causal={causal} {dt}", flush=True)
    g = torch.Generator().manual_seed(sum(lq) * 13 + sum(lk) + D)
    cq = torch.tensor([0] + torch.tensor(lq).cumsum(0).tolist(), dtype=torch.int32)
    ck = torch.tensor([0] + torch.tensor(lk).cumsum(0).tolist(), dtype=torch.int32)
    q = torch.randn(int(cq[-1]), H, D, generator=g).to(dt)
    k = torch.randn(int(ck[-1]), Hkv, D, generator=g).to(dt)
    v = torch.randn(int(ck[-1]), Hkv, D, generator=g).to(dt)
    o = torch.full(tuple(q.shape), float("nan"), dtype=dt, device=DEV)
    sc = 1 / math.sqrt(D)
    ops.flash_attn_varlen_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(lq),
                              o, causal, sc)
    exp = ref.flashattn_varlen_ref(q, k, v, cq, ck, causal, sc, max_seqlen_q=max(lq))
    torch_assert_close(o.cpu().float(), exp, atol=2e-2, rtol=2e-2)


def _splitkv_cases(n, seed):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        ns = r.choice([1, 2, 3, 4, 8])
        Hkv = r.choice([1, 2])
        out.append((r.randint(1, 2), r.choice([1, 16, 100, 128, 129, 300]),
                    ns * 64 * r.choice([1, 2, 5, 16]), Hkv * r.choice([1, 2, 4]), Hkv,
                    r.choice([32, 64, 128]), ns, r.choice([torch.float16, torch.bfloat16])))
    return out


@pytest.mark.parametrize("B,Sq,Sk,H,Hkv,D,ns,dt", _splitkv_cases(8, seed=93))
def test_flashattn_splitkv_random(B, Sq, Sk, H, Hkv, D, ns, dt):
    """Split-KV inference (example_mha_inference.py) over random split counts and lengths: the
    written Output_partial and glse against the restated flash_split_ref, Output against the
    full attention."""
    print(f"splitkv B={B} Sq={Sq} Sk={Sk} H={H} Hkv={Hkv} D={D} ns={ns} {dt}", flush=True)
    g = torch.Generator().manual_seed(B * 101 + Sq * 7 + Sk + D + ns)
    q = torch.randn(B, Sq, H, D, generator=g).to(dt)
    k = torch.randn(B, Sk, Hkv, D, generator=g).to(dt)
    v = torch.randn(B, Sk, Hkv, D, generator=g).to(dt)
    glse = torch.full((B, H, ns, Sq), float("nan"), dtype=dt, device=DEV)
    part = torch.full((B, Sq, H, ns, D), float("nan"), dtype=dt, device=DEV)
    o = torch.full((B, Sq, H, D), float("nan"), dtype=dt, device=DEV)
    ws = torch.empty(ops.flash_attn_splitkv_workspace_bytes(B, Sq, Sk, H, D, ns),
                     dtype=torch.uint8, device=DEV)
    ops.flash_attn_splitkv_fwd(q.to(DEV), k.to(DEV), v.to(DEV), glse, part, o, ns, D ** -0.5, ws)
    kr, vr = k.repeat_interleave(H // Hkv, dim=2), v.repeat_interleave(H // Hkv, dim=2)
    torch_assert_close(o.cpu().float(), ref.mha_inference_ref(q, kr, vr), atol=2e-2, rtol=2e-2)
    _, (g_ref, p_ref) = ref.mha_split_combine_ref(q, kr, vr, ns, 64, store_dtype=dt)
    torch_assert_close(part.cpu().float(), p_ref, atol=2e-2, rtol=2e-2)
    # one ulp of a log2 sum-exp below 32: 2^-6 in fp16, 2^-3 in bf16
    torch_assert_close(glse.cpu().float(), g_ref, atol=0.13 if dt == torch.bfloat16 else 2e-2,
                       rtol=0)
