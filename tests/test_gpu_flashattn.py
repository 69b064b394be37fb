"""GPU parity: FlashAttention forward through ``tilelang.compile`` against the oracle
(restated ref_program, tpu_demo/flashattn/tpu_test_flashattn_bf16.py:171-182).

Tolerance: the demo's atol=rtol=5e-2 (:197) and, tighter, 2e-2 (P is rounded to bf16 before
P@V as in the program, :80, so the kernel cannot match an fp32-P oracle more closely).
Full-size configs are checked on every (batch, head) pair over three 256-query tiles; the oracle
is exact fp32.
"""
import math

import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs, workloads
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_flashattn_demo_program_tpu_convention():
    """The demo's own tiny case: B=1, H=2, S=4, D=8 is not a kernel shape (D in {64,128});
    run the demo flow (CPU tensors, all params, in place) at the smallest supported D."""
    B, H, S, D = 1, 2, 16, 64
    k = tilelang.compile(programs.flashattn(B, H, S, D, False, 2, 2), out_idx=-1, target="tpu")
    w = workloads.flashattn(B, S, H, D, causal=False, seed=21)
    out = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    assert k(w.tensors["q"], w.tensors["k"], w.tensors["v"], out) == 0
    exp = ref.flashattn_ref(w.tensors["q"], w.tensors["k"], w.tensors["v"], False)
    torch_assert_close(out, exp, atol=5e-2, rtol=5e-2)


@pytest.mark.parametrize("B,S,H,D,causal", [
    (2, 256, 2, 128, True), (2, 256, 2, 128, False), (1, 300, 3, 128, True),
    (1, 77, 2, 64, False), (1, 1000, 1, 64, True), (2, 513, 2, 128, False),
])
def test_flashattn_small(B, S, H, D, causal):
    w = workloads.flashattn(B, S, H, D, causal=causal, seed=22)
    k = tilelang.compile(programs.flashattn(B, H, S, D, causal), out_idx=-1)
    o = k(*(w.tensors[n].to(DEV) for n in ("q", "k", "v")))
    exp = ref.flashattn_ref(w.tensors["q"], w.tensors["k"], w.tensors["v"], causal)
    torch_assert_close(o.cpu(), exp, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("S,causal", [(4096, True), (2048, False)])
def test_flashattn_config_all_heads(S, causal):
    """The full config: every (batch, head) pair is compared on the first, a middle and the last
    256-query tile (the workgroup order regroups heads per XCD and pairs causal tiles, so each
    pair maps differently); the output starts as NaN, so a tile the kernel never writes fails."""
    B, H, D = 8, 32, 128
    w = workloads.flashattn(B, S, H, D, causal=causal)
    q, kk, v = (w.tensors[n] for n in ("q", "k", "v"))
    o = torch.full((B, S, H, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    ops.flash_attn_fwd(q.to(DEV), kk.to(DEV), v.to(DEV), o, causal, 1 / math.sqrt(D))
    o = o.cpu()
    assert not torch.isnan(o).any()
    mid = (S // 256 // 2) * 256
    rows = list(range(0, 256)) + list(range(mid, mid + 256)) + list(range(S - 256, S))
    exp = ref.flashattn_rows_ref(q, kk, v, causal, rows)
    torch_assert_close(o[:, rows], exp.to(torch.bfloat16), atol=2e-2, rtol=2e-2)


def test_flashattn_single_key_returns_v():
    """S=1: softmax over one key is 1, so O == V exactly."""
    w = workloads.flashattn(2, 1, 4, 128, causal=True, seed=23)
    o = torch.empty(2, 1, 4, 128, dtype=torch.bfloat16, device=DEV)
    q, kk, v = (w.tensors[n].to(DEV) for n in ("q", "k", "v"))
    ops.flash_attn_fwd(q, kk, v, o, True, 1 / math.sqrt(128))
    assert torch.equal(o, v)


def test_flashattn_fp16_and_consistency():
    w = workloads.flashattn(1, 384, 2, 128, dtype=torch.float16, seed=24)
    k = tilelang.compile(programs.flashattn(1, 2, 384, 128, True, dtype="float16"), out_idx=-1)
    ins = [w.tensors[n].to(DEV) for n in ("q", "k", "v")]
    o1 = k(*ins)
    o2 = k(*ins)
    assert torch.equal(o1, o2)
    exp = ref.flashattn_ref(w.tensors["q"], w.tensors["k"], w.tensors["v"], True)
    torch_assert_close(o1.cpu(), exp, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("D,dtype,causal", [
    (128, torch.bfloat16, True), (128, torch.bfloat16, False), (128, torch.float16, True),
    (128, torch.float16, False), (64, torch.bfloat16, False), (64, torch.float16, False),
    (64, torch.bfloat16, True), (64, torch.float16, True)])
def test_flashattn_score_jumps_rescale(D, dtype, causal):
    """Keys of 64-key tile t scaled by 1 + 30 t: a row's scores have spread ~(1 + 30 t), so the
    tile maximum rises by ~75 nats (~108 log2 units) from tile to tile, past the lazy-max
    headroom of both P limits (2^64 for bf16 P, 2^15 for fp16 P). Every tile after the first is
    then redone against its own maximum with O and l rescaled (the D = 64 non-causal kernel and
    the D = 128 kernel); the D = 64 causal kernel keeps the per-tile maximum."""
    w = workloads.flashattn(1, 640, 2, D, causal=causal, dtype=dtype, seed=25)
    q, kk, v = (w.tensors[n] for n in ("q", "k", "v"))
    f = (1 + 30 * (torch.arange(640) // 64)).to(torch.float32).view(1, 640, 1, 1)
    kk = (kk.float() * f).to(dtype)
    assert torch.isfinite(kk.float()).all()
    o = torch.full(q.shape, float("nan"), dtype=dtype, device=DEV)
    ops.flash_attn_fwd(q.to(DEV), kk.to(DEV), v.to(DEV), o, causal, 1 / math.sqrt(D))
    exp = ref.flashattn_ref(q, kk, v, causal)
    torch_assert_close(o.cpu(), exp, atol=2e-2, rtol=2e-2)
