"""GPU parity: grouped-query FlashAttention forward (examples/flash_attention/example_gqa_fwd_bshd.py)
and the upstream MHA program structure (groups = 1, example_mha_fwd_bshd.py), compiled with
``tilelang.compile`` and checked against the oracle (ref_program of the example, :181-205, with
K/V repeated per group). Tolerance: the example's atol = rtol = 1e-2 (:220), with 2e-2 for the
fp16 P rounding at long sequences; sampled heads at the example's own default size.
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


def _qkv(B, S, H, Hkv, D, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, D, generator=g).to(dtype)
    k = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, S, Hkv, D, generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("B,H,S,D,causal,groups", [
    (1, 8, 512, 128, True, 4),     # tiled D = 128 kernel
    (2, 8, 300, 128, False, 2),    # ragged S
    (1, 16, 640, 128, True, 16),   # one K/V head
    (2, 4, 256, 64, True, 2),      # D = 64 kernel
    (1, 4, 100, 96, False, 2),     # per-query kernel
    (2, 4, 384, 128, True, 1),     # upstream MHA structure
])
def test_gqa_program(B, H, S, D, causal, groups):
    q, k, v = _qkv(B, S, H, H // groups, D, seed=70)
    kern = tilelang.compile(programs.flashattn_gqa(B, H, S, D, causal, groups), out_idx=[3])
    assert kern.plan.attrs["H_kv"] == H // groups
    o = kern(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    exp = ref.flashattn_ref(q, k, v, causal)
    torch_assert_close(o.float(), exp.float(), atol=1e-2, rtol=1e-2)


def test_gqa_example_default_size_sampled():
    """The example's defaults: batch 1, 64 heads, seq 8192, dim 128, 16 groups (4 K/V heads)."""
    B, H, S, D, G = 1, 64, 8192, 128, 16
    q, k, v = _qkv(B, S, H, H // G, D, seed=71)
    o = torch.empty(B, S, H, D, dtype=torch.float16, device=DEV)
    ops.flash_attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), o, False, 1 / math.sqrt(D))
    o = o.cpu()
    for h in (0, 17, 63):  # heads of K/V heads 0, 1, 3
        exp = ref.flashattn_ref(q, k, v, False, heads=[h])
        torch_assert_close(o[:, :, h].float(), exp[:, :, h].float(), atol=2e-2, rtol=2e-2)
    assert torch.isfinite(o.float()).all()


def test_gqa_equals_mha_on_repeated_kv_bitwise():
    """The grouped path reads exactly the K/V rows the MHA path reads after repeat_interleave:
    both launches give identical bits."""
    B, H, S, D, G = 2, 8, 700, 128, 4
    q, k, v = _qkv(B, S, H, H // G, D, seed=72, dtype=torch.bfloat16)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o1 = torch.empty_like(qd)
    o2 = torch.empty_like(qd)
    ops.flash_attn_fwd(qd, kd, vd, o1, True, 1 / math.sqrt(D))
    kr = kd.repeat_interleave(G, dim=2).contiguous()
    vr = vd.repeat_interleave(G, dim=2).contiguous()
    ops.flash_attn_fwd(qd, kr, vr, o2, True, 1 / math.sqrt(D))
    assert torch.equal(o1, o2)
