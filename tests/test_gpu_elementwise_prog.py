"""GPU parity: stand-alone elementwise T.ppl_* programs through ``tilelang.compile`` and the
elementwise register-program kernel (tlm_elementwise).

Programs (restated in tilelang.testing.programs): tpu_demo/ppl/test/exp.py (in place, fp32 and
bf16 as exp_bf16.py), mul_N_1.py (row-broadcast product), elementwise_c.py (scale and shift),
tpu_demo/ppl/elementwise_add_kernel/elementwise_add.py (sum). Each at the demo's own shape (TPU
convention: CPU tensors, all parameters, written in place) and at larger ones.
Oracle: ref.ppl_*_ref (fp32 math, one rounding per tile write). Tolerances: fp32 outputs 2 ulp
(rtol 2.5e-7, the device expf against torch.exp; exactly rounded ops compare bit-exact), bf16
1 ulp (rtol 8e-3).
"""
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import lib, ops
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.mark.parametrize("M,N,bm,bn,dtype", [(10, 2, 5, 1, "float32"), (10, 2, 5, 1, "bfloat16"),
                                             (1000, 300, 100, 30, "float32")])
def test_exp_in_place(M, N, bm, bn, dtype):
    k = tilelang.compile(programs.ppl_exp(M, N, bm, bn, dtype), out_idx=-1, target="tpu")
    x = (torch.randn(M, N, generator=_g(91)) * 3).to(getattr(torch, dtype))
    exp = ref.ppl_exp_ref(x)
    y = x.clone()
    assert k(y) == 0
    tol = 2.5e-7 if dtype == "float32" else 8e-3
    torch_assert_close(y, exp, atol=0, rtol=tol, max_mismatched_ratio=0)


@pytest.mark.parametrize("M,N,blk", [(8192, 8192, 64), (100, 37, 10)])
def test_mul_rows(M, N, blk):
    k = tilelang.compile(programs.ppl_mul_rows(M, N, blk), out_idx=[0])
    a = torch.randn(M, N, generator=_g(92))
    b = torch.randn(M, 1, generator=_g(93))
    c = k(a.to(DEV), b.to(DEV)).cpu()  # inputs only: C is allocated and returned
    assert torch.equal(c, ref.ppl_mul_rows_ref(a, b))


def test_mul_rows_tpu_convention_demo_shape():
    M, N, blk = 8192, 8192, 64
    k = tilelang.compile(programs.ppl_mul_rows(M, N, blk), out_idx=[0], target="tpu")
    a = torch.randn(M, N, generator=_g(94))
    b = torch.randn(M, 1, generator=_g(95))
    c = torch.zeros(M, N)
    assert k(c, a, b) == 0
    assert torch.equal(c, ref.ppl_mul_rows_ref(a, b))


@pytest.mark.parametrize("M,N,bm,bn,dtype", [(16, 4, 4, 2, "float32"), (512, 4096, 64, 64, "float32"),
                                             (256, 256, 32, 32, "bfloat16")])
def test_scale_shift(M, N, bm, bn, dtype):
    k = tilelang.compile(programs.ppl_scale_shift(M, N, bm, bn, dtype), out_idx=-1, target="tpu")
    a = (torch.randn(M, N, generator=_g(96)) * 100).to(getattr(torch, dtype))
    b = torch.zeros(M, N, dtype=a.dtype)
    assert k(a, b) == 0
    assert torch.equal(b, ref.ppl_scale_shift_ref(a, 1 / 8192, 1e-12))


@pytest.mark.parametrize("in_dt,out_dt", [("float32", "float32"), ("float16", "float32"),
                                          ("bfloat16", "bfloat16")])
def test_add(in_dt, out_dt):
    M, N = 512, 1024
    k = tilelang.compile(programs.ppl_add(M, N, 128, 256, in_dt, out_dt), out_idx=-1)
    a = torch.randn(M, N, generator=_g(97)).to(getattr(torch, in_dt))
    b = torch.randn(M, N, generator=_g(98)).to(getattr(torch, in_dt))
    c = k(a.to(DEV), b.to(DEV)).cpu()
    assert torch.equal(c, ref.ppl_add_ref(a, b, getattr(torch, out_dt)))


def test_register_program_through_the_c_abi():
    """A hand-assembled program over every op and broadcast kind (sigmoid(a * row + col) /
    rsqrt(scalar) - 1, exp, rounding to fp16), against the same chain in torch."""
    M, N = 33, 70
    g = _g(99)
    a = torch.randn(M, N, generator=g)
    row = torch.randn(M, 1, generator=g)
    col = torch.randn(1, N, generator=g)
    sc = torch.tensor([4.0])
    E = lambda op, d, x=0, y=0, imm=0: op | d << 8 | x << 12 | y << 16 | imm << 20
    code = [E(lib.EW_LOAD, 0, imm=0), E(lib.EW_LOAD, 1, imm=1), E(lib.EW_MUL, 0, 0, 1),
            E(lib.EW_LOAD, 1, imm=2), E(lib.EW_ADD, 0, 0, 1), E(lib.EW_SIGMOID, 0, 0),
            E(lib.EW_LOAD, 1, imm=3), E(lib.EW_RSQRT, 1, 1), E(lib.EW_DIV, 0, 0, 1),
            E(lib.EW_CONST, 2, imm=0), E(lib.EW_SUB, 0, 0, 2), E(lib.EW_STORE, 0, 0, imm=0),
            E(lib.EW_EXP, 3, 0), E(lib.EW_ROUND, 3, 3, imm=lib.F16), E(lib.EW_STORE, 0, 3, imm=1)]
    o1 = torch.empty(M, N, device=DEV)
    o2 = torch.empty(M, N, dtype=torch.float16, device=DEV)
    ins = [x.to(DEV) for x in (a, row, col, sc)]
    ops.elementwise(ins, [lib.EW_FULL, lib.EW_ROW, lib.EW_COL, lib.EW_SCALAR], [o1, o2], code,
                    [1.0], M, N)
    e1 = torch.sigmoid(a * row + col) / (1.0 / torch.sqrt(sc)) - 1.0
    torch_assert_close(o1.cpu(), e1, atol=1e-6, rtol=1e-6)
    torch_assert_close(o2.cpu().float(), torch.exp(e1).half().float(), atol=0, rtol=1e-3)


def test_symbolic_fill_program_per_binding():
    """tpu_demo/ppl/matmul.py (:9-26) with symbolic m, n: one compiled kernel, called on
    tensors of several shapes (including tiles cut by the edge); every element takes the fill
    value rounded to the tensor's dtype (bit-exact)."""
    import tilelang.language as T
    k = tilelang.compile(programs.fill_tiles(T.symbolic("m"), T.symbolic("n"), 128, 128,
                                             value=0.0), out_idx=-1)
    for (m, n) in ((300, 520), (128, 64), (1, 1000)):
        a = torch.full((m, n), 7.0, dtype=torch.float16, device=DEV)
        assert k(a) == 0
        assert torch.equal(a.cpu(), torch.zeros(m, n, dtype=torch.float16))
    k2 = tilelang.compile(programs.fill_tiles(T.symbolic("m"), T.symbolic("n"), 64, 32,
                                              dtype="bfloat16", value=1.0 / 3), out_idx=-1)
    a = torch.empty(70, 90, dtype=torch.bfloat16, device=DEV)
    assert k2(a) == 0  # the only parameter is the output: all parameters, in place
    exp = torch.full((70, 90), 1.0 / 3, dtype=torch.float32).to(torch.bfloat16)
    assert torch.equal(a.cpu(), exp)
    with pytest.raises(ValueError, match="not bound"):
        k2()  # inputs only: nothing binds m, n


def test_symbolic_add_program_shapes():
    """elementwise_add.py over symbolic m, n: the binding comes from A; B and C must agree."""
    k = tilelang.compile(programs.add_symbolic(64, 64), out_idx=-1)
    for (m, n) in ((100, 70), (256, 512)):
        a = torch.randn(m, n, generator=_g(m)).to(DEV)
        b = torch.randn(m, n, generator=_g(n)).to(DEV)
        c = k(a, b)
        torch_assert_close(c.cpu(), ref.ppl_add_ref(a.cpu(), b.cpu()), atol=0, rtol=0,
                           max_mismatched_ratio=0)
    with pytest.raises(ValueError, match="mismatch"):
        k(torch.zeros(4, 6, device=DEV), torch.zeros(4, 5, device=DEV))
