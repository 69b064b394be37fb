"""GPU parity over seeded random shapes for the tiled MFMA kernels (16x16 operand layouts, LDS
swizzles, edge masking): GEMM (both B layouts, fp16 / bf16, ragged M, N, K), FP8 GEMM and
FlashAttention (causal or not, grouped K/V heads, head dim 64 and 128, ragged S). Each case
prints its shape before it runs. Tolerances follow the family tests: GEMM 1e-2 (the demo's),
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
