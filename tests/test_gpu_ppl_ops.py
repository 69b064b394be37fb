"""GPU parity for the remaining TPU demo ops: sigmoid, gather, topk, row reductions.

Each demo program (tpu_demo/tpu_test_{sigmoid_fp32,gather_fp32,topk_fp32,reduce_max,
reduce_sum}.py) is compiled with ``tilelang.compile`` and run the demo's way (CPU tensors, all
parameters, outputs in place), then the C ABI is exercised at other sizes and edge cases.
Bit-exact: gather (a copy), topk values and indices (a sort), reduce_max. Tolerances: sigmoid
fp32 within 2e-6 absolute (v_exp / v_rcp are within a few ulps; the demo allows 1e-2), 16-bit
sigmoid within one rounding; reduce_sum within one rounding of the fp32 sum.
"""
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_sigmoid_demo():
    C = W = 1024
    a = torch.randn(C, W, generator=_g(90))
    k = tilelang.compile(programs.sigmoid(32, 32, C, W), out_idx=-1, target="tpu")
    out = torch.zeros(C, W)
    assert k(a, out) == 0
    torch_assert_close(out, ref.sigmoid_ref(a), atol=2e-6, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_sigmoid_edges(dtype):
    x = torch.cat([torch.tensor([0.0, -0.0, 1e-8, 88.0, -88.0, 100.0, -100.0, float("inf"),
                                 float("-inf"), float("nan")]),
                   torch.randn(1001, generator=_g(91)) * 10]).to(dtype)  # odd length: scalar tail
    y = torch.empty_like(x, device=DEV)
    ops.sigmoid(x.to(DEV), y)
    got, exp = y.cpu().float(), ref.sigmoid_ref(x).float()
    assert torch.equal(torch.isnan(got), torch.isnan(exp))
    tol = 2e-6 if dtype == torch.float32 else (1e-3 if dtype == torch.float16 else 8e-3)
    torch_assert_close(got, exp, atol=tol, rtol=0, equal_nan=True)


def test_gather_demo():
    param = torch.randn(128, 64, generator=_g(92))
    idx = torch.randint(0, 128, (8, 1), dtype=torch.int32, generator=_g(93))
    k = tilelang.compile(programs.gather(128, 64, 8), out_idx=-1, target="tpu")
    out = torch.zeros(8, 64)
    assert k(param, idx.view(torch.uint32), out) == 0
    assert torch.equal(out, param[idx.view(-1).long()])


@pytest.mark.parametrize("dtype,hidden", [(torch.float32, 576), (torch.bfloat16, 64),
                                          (torch.float16, 33), (torch.float32, 7)])
def test_gather_rows_bit_exact(dtype, hidden):
    """16-byte, 4-byte and 2-byte copy paths; indices past the last row give zero rows."""
    rows, n = 5000, 3001
    param = torch.randn(rows, hidden, generator=_g(94)).to(dtype)
    idx = torch.randint(0, rows, (n,), dtype=torch.int64, generator=_g(95))
    idx[:4] = torch.tensor([rows, rows + 7, 2 ** 32 - 1, 0])
    index = idx.to(torch.uint32)
    out = torch.empty(n, hidden, dtype=dtype, device=DEV)
    ops.gather_rows(param.to(DEV), index.to(DEV), out)
    exp = ref.gather_ref(param, index)
    assert torch.equal(out.cpu().view(torch.uint8), exp.view(torch.uint8))
    assert (out[:3] == 0).all()


def test_topk_demo():
    L, K = 1024, 8
    src = torch.randn(L, generator=_g(96))
    k = tilelang.compile(programs.topk(L, K, True), out_idx=[1, 2], target="tpu")
    vals = torch.zeros(L)
    idxs = torch.zeros(L, dtype=torch.int32)
    assert k(src, vals, idxs) == 0
    rv, ri = torch.topk(src, K, largest=True, sorted=True)
    assert torch.equal(vals[:K], rv) and torch.equal(idxs[:K].long(), ri)
    ev, ei = ref.topk_ref(src, True)
    assert torch.equal(vals, ev) and torch.equal(idxs, ei)


@pytest.mark.parametrize("descending", [True, False])
@pytest.mark.parametrize("L", [1, 2, 3, 1000, 4096, 16384])
def test_topk_full_order_fp32(L, descending):
    """Ties (values drawn from 50 levels), NaN, infinities and signed zeros."""
    src = (torch.randint(0, 50, (L,), generator=_g(97)).float() - 25) / 4
    if L >= 8:
        src[:8] = torch.tensor([float("nan"), -0.0, 0.0, float("inf"), float("-inf"),
                                float("nan"), 0.0, -0.0])
    vals = torch.empty(L, device=DEV)
    idxs = torch.empty(L, dtype=torch.int32, device=DEV)
    ops.topk(src.to(DEV), min(8, L), descending, vals, idxs)
    ev, ei = ref.topk_ref(src, descending)
    assert torch.equal(idxs.cpu(), ei)
    assert torch.equal(vals.cpu().view(torch.int32), ev.view(torch.int32))


@pytest.mark.parametrize("dtype", [torch.int32, torch.uint32])
def test_topk_integers(dtype):
    L = 3000
    raw = torch.randint(-2 ** 31, 2 ** 31, (L,), dtype=torch.int64, generator=_g(98))
    raw[:6] = torch.tensor([-2 ** 31, 2 ** 31 - 1, 0, -1, 5, 5])
    src = raw.to(torch.int32).view(dtype) if dtype == torch.uint32 else raw.to(torch.int32)
    for desc in (True, False):
        vals = torch.empty(L, dtype=dtype, device=DEV)
        idxs = torch.empty(L, dtype=torch.int32, device=DEV)
        ops.topk(src.to(DEV), 5, desc, vals, idxs)
        ev, ei = ref.topk_ref(src, desc)
        assert torch.equal(idxs.cpu(), ei)
        assert torch.equal(vals.cpu().view(torch.int32), ev.view(torch.int32))


@pytest.mark.parametrize("op", ["max", "sum"])
def test_row_reduce_demo(op):
    M, N = 64, 64
    x = torch.randn(M, N, generator=_g(99)).half()
    k = tilelang.compile(programs.row_reduce(M, N, 32, 64, op), out_idx=-1, target="tpu")
    y = torch.zeros(M, 1).half()
    assert k(x, y) == 0
    exp = torch.max(x, dim=1, keepdim=True).values if op == "max" else ref.row_reduce_ref(x, op)
    if op == "max":
        assert torch.equal(y, exp)
    else:  # the fp32 sum rounded once: within one fp16 rounding of the oracle
        torch_assert_close(y.float(), exp.float(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("in_dt,out_dt", [(torch.float32, torch.float32),
                                          (torch.bfloat16, torch.float32),
                                          (torch.float16, torch.bfloat16)])
def test_row_reduce_shapes(in_dt, out_dt):
    M, N = 777, 1001
    x = torch.randn(M, N, generator=_g(100)).to(in_dt)
    x[5, 17] = float("nan")
    for op in ("max", "sum"):
        y = torch.empty(M, 1, dtype=out_dt, device=DEV)
        ops.row_reduce(x.to(DEV), y, op)
        exp = ref.row_reduce_ref(x, op, out_dt)
        got = y.cpu()
        assert torch.isnan(got[5]).all() and torch.equal(torch.isnan(got), torch.isnan(exp))
        if op == "max":
            assert torch.equal(got[~torch.isnan(exp)], exp[~torch.isnan(exp)])
        else:
            torch_assert_close(got.float(), exp.float(), atol=2e-3, rtol=8e-3, equal_nan=True)
