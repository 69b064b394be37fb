"""GPU parity: head-major FlashAttention (examples/flash_attention/example_mha_fwd_bhsd.py)
through ``tilelang.compile`` and the C ABI, against oracle.ref.flashattn_bhsd_ref (fp32).

Tolerances: the example's own check, atol = rtol = 1e-2 (:215), for fp16; 2e-2 for bf16 (P is
rounded to the input type before P V, as the program's acc_s_cast, so the kernel cannot follow
an fp32-P oracle more closely). At S_q == S_kv the head-major launch must equal the
sequence-major one on transposed tensors bit for bit (same tiles, same order).
"""
import math

import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qkv(B, H, Hkv, Sq, Sk, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Sq, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, Sk, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, Sk, D, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("causal", [False, True])
def test_example_program_defaults(causal):
    """The example's defaults: batch 1, heads 1, seq_q = seq_kv = 256, dim 64, fp16."""
    B, H, S, D = 1, 1, 256, 64
    q, k, v = _qkv(B, H, H, S, S, D, torch.float16, seed=70)
    kern = tilelang.compile(programs.flashattn_bhsd(B, H, S, S, D, causal), out_idx=[3])
    out = kern(q.to(DEV), k.to(DEV), v.to(DEV))
    assert out.shape == q.shape and out.dtype == torch.float16
    exp = ref.flashattn_bhsd_ref(q, k, v, causal)
    torch_assert_close(out.cpu().float(), exp, atol=1e-2, rtol=1e-2)


def test_program_unequal_lengths():
    """seq_q != seq_kv through the program (non-causal, the form the example defines there)."""
    B, H, Sq, Sk, D = 2, 4, 300, 1000, 128
    q, k, v = _qkv(B, H, H, Sq, Sk, D, torch.float16, seed=71)
    kern = tilelang.compile(programs.flashattn_bhsd(B, H, Sq, Sk, D, False), out_idx=[3])
    out = kern(q.to(DEV), k.to(DEV), v.to(DEV))
    torch_assert_close(out.cpu().float(), ref.flashattn_bhsd_ref(q, k, v, False), atol=1e-2,
                       rtol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,Sk", [(300, 1000), (1000, 300), (65, 513), (257, 257)])
@pytest.mark.parametrize("D,Hkv", [(128, 2), (64, 8), (32, 2)])
def test_bhsd_lengths_and_heads(dtype, causal, Sq, Sk, D, Hkv):
    """Unequal and ragged lengths around the 64-key tile and 256-query workgroup edges, grouped
    K/V heads; causal keeps key j <= i + S_kv - S_q (rows without a key are zero). D = 128 and
    64 run the tiled MFMA kernels, D = 32 the per-query kernel."""
    print(f"bhsd Sq={Sq} Sk={Sk} D={D} Hkv={Hkv} causal={causal} {dtype}", flush=True)
    B, H = 2, 8
    q, k, v = _qkv(B, H, Hkv, Sq, Sk, D, dtype, seed=Sq + Sk + D)
    o = torch.full(q.shape, 7.0, dtype=dtype, device=DEV)
    sc = 1 / math.sqrt(D)
    ops.flash_attn_bhsd_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, causal, sc)
    exp = ref.flashattn_bhsd_ref(q, k, v, causal, sc)
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    torch_assert_close(o.cpu().float(), exp, atol=tol, rtol=tol)


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_bhsd_equals_bshd_bitwise(D, causal):
    B, H, Hkv, S = 2, 8, 4, 600
    q, k, v = (t.to(DEV) for t in _qkv(B, H, Hkv, S, S, D, torch.bfloat16, seed=72))
    o = torch.empty_like(q)
    ops.flash_attn_bhsd_fwd(q, k, v, o, causal, 0.1)
    qs, ks, vs = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    os_ = torch.empty_like(qs)
    ops.flash_attn_fwd(qs, ks, vs, os_, causal, 0.1)
    assert torch.equal(o, os_.transpose(1, 2))


def test_fp32_output_and_rows_without_keys():
    B, H, Sq, D = 1, 4, 200, 128
    q, k, v = _qkv(B, H, H, Sq, 150, D, torch.float16, seed=73)
    o = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    ops.flash_attn_bhsd_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, True, 0.09)
    exp = ref.flashattn_bhsd_ref(q, k, v, True, 0.09)
    torch_assert_close(o.cpu(), exp, atol=1e-2, rtol=1e-2)
    assert torch.equal(o[:, :, :50].cpu(), torch.zeros(B, H, 50, D))  # 50 queries see no key
