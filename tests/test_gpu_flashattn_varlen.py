"""GPU parity: variable-length FlashAttention (examples/flash_attention/example_mha_fwd_varlen.py)
through ``tilelang.compile`` and the C ABI, against oracle.ref.flashattn_varlen_ref (fp32).

Tolerances: the example's own check, atol = rtol = 1e-2 (:440), for fp16; 2e-2 for bf16 (P is
rounded to the input type before P V, as the program's acc_s_cast, :335, so the kernel cannot
follow an fp32-P oracle more closely). Equal-length batches must equal the dense kernel bit for
bit (same tiles, same order).
"""
import math

import numpy as np
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lens_q, lens_k, H, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    cu_q = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), H, D, generator=g).to(dtype)
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dtype)
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).to(dtype)
    return q, k, v, cu_q, cu_k


def _check(o, exp, cu_q, tol):
    """Compare the rows the oracle defines (it leaves unwritten rows NaN)."""
    rows = ~torch.isnan(exp).any(dim=2).any(dim=1)
    assert rows.any()
    torch_assert_close(o.cpu().float()[rows], exp[rows], atol=tol, rtol=tol)


def test_example_program_defaults():
    """The example's defaults: batch 2, 16 heads, seq 256, dim 32, fp16, padding masks of mode
    "random" (lengths in [seq - 20, seq], :20-21) on both sides, max_seqlen_q from the queries."""
    B, H, S, D = 2, 16, 256, 32
    g = torch.Generator().manual_seed(60)
    lq = torch.randint(S - 20, S + 1, (B,), generator=g).tolist()
    lk = torch.randint(S - 20, S + 1, (B,), generator=g).tolist()
    q, k, v, cu_q, cu_k = _case(lq, lk, H, H, D, torch.float16, seed=61)
    kern = tilelang.compile(programs.flashattn_varlen(B, q.shape[0], k.shape[0], H, D),
                            out_idx=-1)
    out = kern(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV), max(lq))
    assert out.shape == q.shape and out.dtype == torch.float16
    exp = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, sm_scale=1 / math.sqrt(D))
    _check(out, exp, cu_q, 1e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D,Hkv", [(128, 4), (128, 1), (64, 2), (32, 4)])
def test_ragged_lengths(dtype, causal, D, Hkv):
    """Lengths around the 64-key tile and 256-query workgroup edges, a one-token sequence, an
    empty query side and an empty key side; grouped K/V heads; D = 128 and 64 run the tiled MFMA
    kernels, other dims the per-query kernel."""
    lens_q = [1, 63, 257, 0, 300, 5, 130]
    lens_k = [70, 64, 257, 10, 1000, 0, 65]
    H = 4
    q, k, v, cu_q, cu_k = _case(lens_q, lens_k, H, Hkv, D, dtype, seed=62)
    o = torch.full(q.shape, 7.0, dtype=dtype, device=DEV)
    sc = 1 / math.sqrt(D)
    ops.flash_attn_varlen_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                              max(lens_q), o, causal, sc)
    exp = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, causal, sc)
    _check(o, exp, cu_q, 1e-2 if dtype == torch.float16 else 2e-2)
    # the sequence without keys gives zero rows (5 queries after cu_q[5])
    assert torch.equal(o[int(cu_q[5]):int(cu_q[6])].cpu().float(), torch.zeros(5, H, D))


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_equal_lengths_match_dense_kernel_bitwise(D, causal):
    B, S, H = 3, 300, 4
    q, k, v, cu_q, cu_k = _case([S] * B, [S] * B, H, H, D, torch.bfloat16, seed=63)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o_var = torch.empty_like(qd)
    ops.flash_attn_varlen_fwd(qd, kd, vd, cu_q.to(DEV), cu_k.to(DEV), S, o_var, causal, 0.1)
    o_dense = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=DEV)
    ops.flash_attn_fwd(qd.view(B, S, H, D), kd.view(B, S, H, D), vd.view(B, S, H, D), o_dense,
                       causal, 0.1)
    assert torch.equal(o_var.view(B, S, H, D), o_dense)  # the same tiled kernel and tile order


def test_fp32_output_and_untouched_rows():
    """fp32 output; queries at positions >= max_seqlen_q and a sequence whose offsets run past
    the tensors are not written (the output keeps its sentinel)."""
    H, D = 2, 128
    lens_q, lens_k = [40, 300, 20], [50, 280, 30]
    q, k, v, cu_q, cu_k = _case(lens_q, lens_k, H, H, D, torch.float16, seed=64)
    o = torch.full(q.shape, -3.0, dtype=torch.float32, device=DEV)
    ops.flash_attn_varlen_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV), 256,
                              o, False, 0.08)
    exp = ref.flashattn_varlen_ref(q, k, v, cu_q, cu_k, False, 0.08, max_seqlen_q=256)
    _check(o, exp, cu_q, 1e-2)
    assert (o[40 + 256:340].cpu() == -3.0).all()  # positions 256..299 of sequence 1
    # sequence 2 claims key rows past total_k: skipped, its output rows keep the sentinel
    bad_k = cu_k.clone()
    bad_k[3] = int(cu_k[3]) + 5
    o2 = torch.full(q.shape, -3.0, dtype=torch.float32, device=DEV)
    ops.flash_attn_varlen_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), bad_k.to(DEV), 300,
                              o2, False, 0.08)
    assert (o2[340:].cpu() == -3.0).all()
    torch.testing.assert_close(o2[:340].cpu(), ops_full(q, k, v, cu_q, cu_k)[:340], atol=0,
                               rtol=0)


def ops_full(q, k, v, cu_q, cu_k):
    o = torch.full(q.shape, -3.0, dtype=torch.float32, device=DEV)
    ops.flash_attn_varlen_fwd(q.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), cu_k.to(DEV), 300,
                              o, False, 0.08)
    return o.cpu()
