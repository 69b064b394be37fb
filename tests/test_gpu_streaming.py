"""GPU parity: RMSNorm, SwiGLU, RoPE through ``tilelang.compile(..., target="mi355x")``
against the CPU oracle on identical seeded inputs.

Tolerances: the demos' own (rms_norm_fp16.py:66 atol=rtol=5e-2; tpu_test_rope_bf16.py:135 and
tpu_test_swiglu_bf16.py:79 atol=rtol=1e-2) and, tighter, a bound of about one rounding step of the
output format against the fp32-evaluated oracle.
"""
import pytest
import torch

import tilelang
from tilelang.testing import programs, workloads
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulp_close(out, exp, rel):
    torch_assert_close(out.cpu(), exp.cpu(), rtol=rel, atol=rel, max_mismatched_ratio=0.0)


# ---------------------------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_rmsnorm_demo_program_tpu_convention(dtype):
    """tpu_demo/rms_norm/rms_norm_fp16.py flow: CPU tensors, all params, output in place."""
    M, N = 128, 128
    k = tilelang.compile(programs.rms_norm(M, N, 32, dtype), out_idx=-1, target="tpu")
    td = getattr(torch, dtype)
    a = torch.randn(M, N, generator=torch.Generator().manual_seed(1)).to(td)
    b = torch.zeros(M, N, dtype=td)
    assert k(a, b) == 0
    exp = ref.rmsnorm_ref(a, None, 1e-12)
    torch_assert_close(b, exp, atol=5e-2, rtol=5e-2)
    _ulp_close(b, exp, 8e-3 if dtype == "bfloat16" else 1e-3)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (37, 4096), (5, 8192), (3, 1000), (7, 24),
                                       (1, 512)])
def test_rmsnorm_weight_shapes(rows, cols):
    w = workloads.rmsnorm(rows, cols, seed=2)
    k = tilelang.compile(programs.rms_norm(rows, cols, 1, "float16", eps=1e-6, with_weight=True),
                         out_idx=-1, target="mi355x")
    x, wt = w.tensors["x"].to(DEV), w.tensors["w"].to(DEV)
    y = k(x, wt)  # GPU convention: inputs only, output allocated
    exp = ref.rmsnorm_ref(w.tensors["x"], w.tensors["w"], 1e-6)
    torch_assert_close(y.cpu(), exp, atol=5e-2, rtol=5e-2)
    _ulp_close(y, exp, 2e-3)


def test_rmsnorm_consistent():
    k = tilelang.compile(programs.rms_norm(256, 4096, 1, "float16"), out_idx=-1)
    k.get_profiler().assert_consistent(repeat=3)


# ---------------------------------------------------------------------------------------- SwiGLU
def test_swiglu_demo_program():
    k = tilelang.compile(programs.swi_glu(32, 32, 64, 64), out_idx=-1, target="tpu")
    g = torch.Generator().manual_seed(3)
    a = torch.randn(64, 64, generator=g, dtype=torch.bfloat16)
    b = torch.randn(64, 64, generator=g, dtype=torch.bfloat16)
    c = torch.zeros(64, 64, dtype=torch.bfloat16)
    assert k(a, b, c) == 0
    exp = ref.swiglu_ref(a, b)
    torch_assert_close(c, exp, atol=1e-2, rtol=1e-2)
    _ulp_close(c, exp, 8e-3)


@pytest.mark.parametrize("rows,cols,dtype", [(8192, 14336, "bfloat16"), (3, 7, "bfloat16"),
                                             (129, 1000, "float16")])
def test_swiglu_shapes(rows, cols, dtype):
    td = getattr(torch, dtype)
    w = workloads.swiglu(rows, cols, dtype=td, seed=4)
    k = tilelang.compile(programs.swi_glu(32, 32, rows, cols, dtype), out_idx=-1)
    out = k(w.tensors["gate"].to(DEV), w.tensors["up"].to(DEV))
    exp = ref.swiglu_ref(w.tensors["gate"], w.tensors["up"])
    torch_assert_close(out.cpu(), exp, atol=1e-2, rtol=1e-2)
    _ulp_close(out, exp, 8e-3 if dtype == "bfloat16" else 1e-3)


# ------------------------------------------------------------------------------------------ RoPE
def test_rope_demo_program():
    C, W = 128, 64
    k = tilelang.compile(programs.rope(64, 16, C, W), out_idx=-1, target="tpu")
    x = torch.randn(C, W, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    cos, sin = ref.rope_cos_sin(C, W)
    out = torch.zeros(C, W, dtype=torch.bfloat16)
    assert k(x, cos, sin, out) == 0
    exp = ref.rope_ref(x, cos, sin)
    torch_assert_close(out, exp, atol=1e-2, rtol=1e-2)
    _ulp_close(out, exp, 8e-3)


@pytest.mark.parametrize("tokens,hq,hk,dim", [(8192, 32, 32, 128), (33, 5, 3, 128), (17, 4, 2, 64),
                                              (9, 3, 1, 40)])
def test_rope_qk(tokens, hq, hk, dim):
    w = workloads.rope(tokens, hq, dim, seed=6)
    kk = torch.randn(tokens, hk, dim, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    prog = programs.rope_qk(tokens, hq, hk, dim)
    k = tilelang.compile(prog, out_idx=[4, 5])
    q_out, k_out = k(w.tensors["q"].to(DEV), kk.to(DEV), w.tensors["cos"].to(DEV),
                     w.tensors["sin"].to(DEV))
    eq = ref.rope_ref(w.tensors["q"], w.tensors["cos"], w.tensors["sin"])
    ek = ref.rope_ref(kk, w.tensors["cos"], w.tensors["sin"])
    torch_assert_close(q_out.cpu(), eq, atol=1e-2, rtol=1e-2)
    _ulp_close(q_out, eq, 8e-3)
    _ulp_close(k_out, ek, 8e-3)


def test_rope_output_first_program():
    """tpu_demo/ppl/rope/rope_bf16.py:8-13 order (G_out, G_in, G_cos, G_sin), TPU convention."""
    C, W = 128, 64
    k = tilelang.compile(programs.rope(64, 16, C, W, out_first=True), out_idx=[0], target="tpu")
    x = torch.randn(C, W, generator=torch.Generator().manual_seed(15)).to(torch.bfloat16)
    cos, sin = ref.rope_cos_sin(C, W)
    out = torch.zeros(C, W, dtype=torch.bfloat16)
    assert k(out, x, cos, sin) == 0
    exp = ref.rope_ref(x, cos, sin)
    torch_assert_close(out, exp, atol=1e-2, rtol=1e-2)
    _ulp_close(out, exp, 8e-3)


@pytest.mark.parametrize("tokens,hq,hk,dim", [(40, 4, 2, 128), (9, 3, 1, 40)])
def test_rope_unpaired_tables(tokens, hq, hk, dim):
    """Tables whose even and odd entries differ: the odd output takes cos[2i+1] and the even
    output sin[2i+1], as ppl_rope_add's strided adds do (16-byte and scalar kernels)."""
    g = torch.Generator().manual_seed(16)
    q = torch.randn(tokens, hq, dim, generator=g).to(torch.bfloat16)
    kk = torch.randn(tokens, hk, dim, generator=g).to(torch.bfloat16)
    cos, sin = (torch.randn(tokens, dim, generator=g).to(torch.bfloat16) for _ in range(2))
    k = tilelang.compile(programs.rope_qk(tokens, hq, hk, dim), out_idx=[4, 5])
    q_out, k_out = k(q.to(DEV), kk.to(DEV), cos.to(DEV), sin.to(DEV))
    for got, x in ((q_out, q), (k_out, kk)):
        exp = ref.rope_ref(x, cos, sin)
        torch_assert_close(got.cpu(), exp, atol=2e-2, rtol=8e-3)


def test_rope_position_zero_is_identity():
    w = workloads.rope(4, 8, 128, seed=8)
    k = tilelang.compile(programs.rope_qk(4, 8, 8, 128), out_idx=[4, 5])
    qo, ko = k(*(w.tensors[n].to(DEV) for n in ("q", "k", "cos", "sin")))
    assert torch.equal(qo[0].cpu(), w.tensors["q"][0])
    assert torch.equal(ko[0].cpu(), w.tensors["k"][0])
