"""GPU parity for the remaining tpu_demo programs: fp32 / fp16 twins and split-K RMSNorm.

Each case compiles the program with ``tilelang.compile`` and runs it the way the demo does
(CPU tensors, all parameters, output written in place) or with device tensors, then compares
with the oracle restatement of the demo's torch reference:
  rms_norm/rmsnorm_fp32.py, rmsnorm_splitk_{fp16,bf16,fp32}.py  -> oracle.ref.rmsnorm_ref
  matmul/tpu_test_matmul_fp32.py (fp32 A/B copied to fp16 tiles) -> matmul_ref on fp16-rounded A/B
  tpu_test_rope_{fp16,fp32}.py, tpu_test_rope.py                 -> rope_ref
  tpu_test_swiglu_fp32.py                                        -> swiglu_ref
  flashattn/tpu_test_flashattn_{bf16,fp16,fp32}.py at the demos' own shape (dim 8, seq 4)
                                                                 -> flashattn_ref
Tolerances: fp32 streaming results within 1e-5 relative (v_rcp / v_exp / v_rsq are within a few
ulps); fp16 / bf16 results within the demos' 1e-2; the fp32 programs with fp16 matrix tiles
within 2e-3 of the oracle on the same fp16-rounded operands and within the demos' own 1e-2 of
their all-fp32 torch reference. tlm_cast is bit-exact against torch's round-to-nearest-even.
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


def _gen(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.float16),
                                     (torch.float32, torch.bfloat16),
                                     (torch.float16, torch.float32),
                                     (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("n", [4096, 1000])  # vector path / scalar path
def test_cast_bit_exact(src, dst, n):
    g = _gen(60)
    x = torch.randn(n, generator=g) * torch.exp(torch.randn(n, generator=g) * 8)
    x[:12] = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 65504.0, 65520.0, 1e-8,
                           -6e-8, 3.0e38, 2 ** -24, 1 + 2 ** -11, 1 + 3 * 2 ** -11])
    x = x.to(src)
    y = torch.empty(n, dtype=dst, device=DEV)
    ops.cast(x.to(DEV), y)
    exp = x.to(dst)
    got = y.cpu()
    nan = torch.isnan(exp)
    assert torch.equal(torch.isnan(got), nan)
    bits = torch.int16 if dst != torch.float32 else torch.int32
    assert torch.equal(got[~nan].view(bits), exp[~nan].view(bits))


@pytest.mark.parametrize("M,N", [(128, 512), (64, 4096), (33, 1000)])
def test_rmsnorm_fp32(M, N):
    x = torch.randn(M, N, generator=_gen(61))
    k = tilelang.compile(programs.rms_norm(M, N, 32 if M % 32 == 0 else 1, dtype="float32"),
                         out_idx=-1, target="tpu")
    y = torch.zeros(M, N)
    assert k(x, y) == 0  # the demo flow: CPU tensors, all params, in place
    torch_assert_close(y, ref.rmsnorm_ref(x, None, 1e-12), atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("dtype,tol", [("float16", 5e-2), ("bfloat16", 5e-2), ("float32", 1e-5)])
def test_rmsnorm_splitk(dtype, tol):
    tdt = getattr(torch, dtype)
    M, N = 512, 512
    x = torch.randn(M, N, generator=_gen(62)).to(tdt)
    k = tilelang.compile(programs.rms_norm_splitk(M, N, 32, 32, dtype), out_idx=-1, target="tpu")
    y = k(x.to(DEV)).cpu()
    exp = ref.rmsnorm_ref(x, None, 1e-12)
    torch_assert_close(y, exp, atol=tol, rtol=tol)
    if dtype != "float32":  # one rounding from the same fp32 value: within one ulp
        torch_assert_close(y.float(), exp.float(), atol=1e-2, rtol=8e-3)


@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (256, 320, 512)])
def test_matmul_fp32_program(M, N, K):
    g = _gen(63)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(K, N, generator=g)
    k = tilelang.compile(programs.matmul(M, N, K, 32, 32, 32, "float32", "float32",
                                         operand_dtype="float16"), out_idx=-1, target="tpu")
    c = torch.zeros(M, N)
    assert k(a, b, c) == 0
    exp = ref.matmul_ref(a.half(), b.half(), out_dtype=torch.float32)  # the fp16 tiles
    torch_assert_close(c, exp, atol=2e-3, rtol=2e-3)
    if K == 64:  # the demo's own check against an all-fp32 matmul (tpu_test_matmul_fp32.py:58)
        torch_assert_close(c, a @ b, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-5), ("float16", 1e-2)])
@pytest.mark.parametrize("C,W", [(128, 64), (100, 30)])
def test_rope_fp32_fp16(dtype, tol, C, W):
    tdt = getattr(torch, dtype)
    x = torch.randn(C, W, generator=_gen(64)).to(tdt)
    cos, sin = ref.rope_cos_sin(C, W, dtype=tdt)
    k = tilelang.compile(programs.rope(64, 16, C, W, dtype=dtype), out_idx=-1, target="tpu")
    out = torch.zeros(C, W, dtype=tdt)
    assert k(x, cos, sin, out) == 0
    torch_assert_close(out, ref.rope_ref(x, cos, sin), atol=tol, rtol=tol)
    # tables whose even and odd entries differ (ppl_rope_add's strided adds), output first
    # (tpu_demo/ppl/rope/rope_{fp16,fp32}.py:8-13)
    cos, sin = (torch.randn(C, W, generator=_gen(67)).to(tdt) for _ in range(2))
    k = tilelang.compile(programs.rope(64, 16, C, W, dtype=dtype, out_first=True), out_idx=[0],
                         target="tpu")
    out = torch.zeros(C, W, dtype=tdt)
    assert k(out, x, cos, sin) == 0
    torch_assert_close(out, ref.rope_ref(x, cos, sin), atol=3 * tol, rtol=tol)


@pytest.mark.parametrize("C,W", [(1024, 1024), (37, 11)])
def test_swiglu_fp32(C, W):
    g = _gen(65)
    a = torch.randn(C, W, generator=g)
    b = torch.randn(C, W, generator=g)
    k = tilelang.compile(programs.swi_glu(32, 32, C, W, dtype="float32"), out_idx=-1)
    out = k(a.to(DEV), b.to(DEV)).cpu()
    torch_assert_close(out, ref.swiglu_ref(a, b), atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("causal", [False, True])
def test_flashattn_demo_shape(dtype, causal):
    """The FA demos' own configuration: batch 1, heads 2, seq 4, dim 8."""
    B, H, S, D = 1, 2, 4, 8
    g = _gen(66)
    q, kk, v = (torch.randn(B, S, H, D, generator=g) for _ in range(3))
    if dtype == "float32":
        prog = programs.flashattn(B, H, S, D, causal, 2, 2, dtype="float32", gemm_dtype="float16")
        ops_in = (q, kk, v)
        exp = ref.flashattn_ref(*(t.half().float() for t in (q, kk, v)), causal)  # fp16 tiles
        tol = 2e-3
    else:
        tdt = getattr(torch, dtype)
        q, kk, v = (t.to(tdt) for t in (q, kk, v))
        prog = programs.flashattn(B, H, S, D, causal, 2, 2, dtype=dtype)
        ops_in = (q, kk, v)
        exp = ref.flashattn_ref(q, kk, v, causal).to(tdt)
        tol = 1e-2
    k = tilelang.compile(prog, out_idx=-1, target="tpu")
    out = torch.zeros(B, S, H, D, dtype=ops_in[0].dtype)
    assert k(*ops_in, out) == 0
    torch_assert_close(out.float(), exp.float(), atol=tol, rtol=tol)


@pytest.mark.parametrize("D,S,causal", [(96, 300, True), (256, 130, False), (32, 1000, True),
                                        (8, 257, False)])
def test_flashattn_other_head_dims(D, S, causal):
    """Head dims without a tiled kernel run the per-query kernel (bf16 in / out)."""
    B, H = 2, 3
    g = _gen(67)
    q, kk, v = (torch.randn(B, S, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    o = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=DEV)
    ops.flash_attn_fwd(q.to(DEV), kk.to(DEV), v.to(DEV), o, causal, 1 / math.sqrt(D))
    torch_assert_close(o.cpu().float(), ref.flashattn_ref(q, kk, v, causal).float(), atol=2e-2,
                       rtol=2e-2)


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_flashattn_fp32_output(D, causal):
    """16-bit Q/K/V with fp32 O (the fp32 program after its tile casts): the tiled kernel's
    fp32 epilogue at D = 128, the per-query kernel at D = 64."""
    B, S, H = 1, 384, 2
    g = _gen(68)
    q, kk, v = (torch.randn(B, S, H, D, generator=g) for _ in range(3))
    k = tilelang.compile(programs.flashattn(B, H, S, D, causal, dtype="float32",
                                            gemm_dtype="float16"), out_idx=-1)
    o = k(q.to(DEV), kk.to(DEV), v.to(DEV)).cpu()
    assert o.dtype == torch.float32
    exp = ref.flashattn_ref(*(t.half().float() for t in (q, kk, v)), causal)
    torch_assert_close(o, exp, atol=2e-3, rtol=2e-3)
    # the output is not rounded to fp16: it differs from its own fp16 rounding
    assert not torch.equal(o, o.half().float())


@pytest.mark.parametrize("B,H,S,D,causal", [(1, 2, 4, 8, False), (1, 2, 4, 8, True),
                                            (2, 3, 300, 64, True), (1, 2, 257, 128, False),
                                            (2, 2, 65, 20, False)])
def test_flashattn_all_fp32_program(B, H, S, D, causal):
    """tpu_demo/ppl/flashattn/fa_fp32.py: fp32 Q, K, V, score and P tiles multiplied by ppl_gemm
    in fp32 (no 16-bit rounding anywhere), fp32 output; its own shape is flashattn(1, 2, 4, 8,
    False) with block 2 x 2. TPU convention (CPU tensors, all params, in place). Tolerance
    1e-4: fp32 throughout, against the fp32 oracle."""
    g = _gen(69 + S)
    q, kk, v = (torch.randn(B, S, H, D, generator=g) for _ in range(3))
    k = tilelang.compile(programs.flashattn(B, H, S, D, causal, 2, 2, dtype="float32"),
                         out_idx=-1, target="tpu")
    assert k.plan.attrs["operand_dtype"] is None and k.plan.attrs["dtype"] == "float32"
    out = torch.zeros(B, S, H, D, dtype=torch.float32)
    assert k(q, kk, v, out) == 0
    torch_assert_close(out, ref.flashattn_ref(q, kk, v, causal), atol=1e-4, rtol=1e-4)
