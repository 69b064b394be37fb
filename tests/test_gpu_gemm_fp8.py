"""GPU parity: FP8 GEMM (examples/gemm_fp8/example_tilelang_gemm_fp8.py, _2xAcc.py) through
``tilelang.compile`` and the C ABI, against oracle.ref.gemm_fp8_ref (exact fp8 decode, fp32
accumulation).

Tolerances: fp32 output within 1e-4 relative + 1e-2 absolute (every fp8 product is exact in fp32;
only the summation order differs: two fp32 sums of K = 1024 products with partial sums up to
~128 can differ by K * ulp(128) ~ 8e-3); fp8 output: the example's own check calc_diff < 1e-3
(:31-35, :56), every element within one fp8 step of the oracle's cast, and at least 99% of codes
equal (a different summation order moves values across a rounding boundary now and then).
"""
import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP8 = {"e4m3_float8": torch.float8_e4m3fn, "e5m2_float8": torch.float8_e5m2}


def _ab(M, N, K, dt, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(M, K, generator=g) * scale).to(dt)
    b = (torch.randn(N, K, generator=g) * scale).to(dt)
    return a, b


def calc_diff(x, y):  # the example's similarity measure
    x, y = x.double(), y.double()
    return 1 - 2 * (x * y).sum() / (x * x + y * y).sum()


def _fp8_close(got, exp_f32, dt):
    exp = exp_f32.to(dt)
    g, e = got.float(), exp.float()
    nan = torch.isnan(e)
    assert torch.equal(torch.isnan(g), nan)
    step = 2.0 ** (-3 if dt == torch.float8_e4m3fn else -2)  # relative spacing of the codes
    diff = ~nan & (g != e)  # equal values (including equal infinities) need no bound
    assert torch.isfinite(g[diff]).all() and torch.isfinite(e[diff]).all()
    assert ((g[diff] - e[diff]).abs() <= step * e[diff].abs() + 2.0 ** -9).all()
    assert (got.view(torch.uint8) == exp.view(torch.uint8)).float().mean() > 0.99


@pytest.mark.parametrize("dtype", ["e4m3_float8", "e5m2_float8"])
def test_example_fp8_output(dtype):
    """The example's own test: 1024^3, C in the input fp8 format."""
    dt = FP8[dtype]
    a, b = _ab(1024, 1024, 1024, dt, seed=80)
    k = tilelang.compile(programs.matmul_fp8(1024, 1024, 1024, 128, 128, 64, dtype), out_idx=-1)
    c = k(a.to(DEV), b.to(DEV)).cpu()
    assert c.dtype == dt
    exp = ref.gemm_fp8_ref(a, b)
    assert calc_diff(c.float(), exp.to(dt).float()) < 1e-3
    _fp8_close(c, exp, dt)


@pytest.mark.parametrize("dtype", ["e4m3_float8", "e5m2_float8"])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (300, 200, 600), (512, 768, 4096)])
def test_2xacc_fp32_output(dtype, M, N, K):
    """K tiles of 64 folded every second tile: an even tile count (600 -> 10, ragged last
    tile), so the program's last fold takes the last tile."""
    dt = FP8[dtype]
    a, b = _ab(M, N, K, dt, seed=81)
    k = tilelang.compile(programs.matmul_fp8(M, N, K, 128, 128, 64, dtype, two_acc=True),
                         out_idx=-1)
    c = k(a.to(DEV), b.to(DEV)).cpu()
    assert c.dtype == torch.float32
    torch.testing.assert_close(c, ref.gemm_fp8_ref(a, b), rtol=1e-4, atol=1e-2)


@pytest.mark.parametrize("M,N,K,trans_b", [(16, 300, 256, True), (100, 70, 100, True),
                                           (64, 96, 128, False)])
def test_fallback_shapes(M, N, K, trans_b):
    """Shapes outside the tiled kernel (M <= 16, K % 16 != 0, row-major B) take the per-output
    kernel."""
    dt = torch.float8_e4m3fn
    a, bnk = _ab(M, N, K, dt, seed=82)
    b = bnk if trans_b else bnk.float().t().contiguous().to(dt)
    c = torch.empty(M, N, dtype=torch.float32, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c, trans_b=trans_b)
    torch.testing.assert_close(c.cpu(), ref.gemm_fp8_ref(a, bnk), rtol=1e-4, atol=1e-2)


@pytest.mark.parametrize("out", [torch.float16, torch.bfloat16])
def test_16bit_outputs(out):
    dt = torch.float8_e5m2
    a, b = _ab(512, 512, 512, dt, seed=83)
    c = torch.empty(512, 512, dtype=out, device=DEV)
    ops.gemm(a.to(DEV), b.to(DEV), c, trans_b=True)
    exp = ref.gemm_fp8_ref(a, b)
    torch.testing.assert_close(c.cpu().float(), exp.to(out).float(), rtol=1e-2, atol=1e-2)


def test_fp8_output_overflow_matches_torch_cast():
    """Exact sums, so summation order cannot matter: row i of A and row j of B hold x_i and y_j
    in 29 of their 128 k (zeros elsewhere), C = 29 x_i y_j exactly. The fp8 C equals torch's cast
    code for code: round to nearest even (29 * 4 * 4 = 464 is the e4m3 tie that rounds to 448),
    no saturation (e4m3 beyond 464 -> NaN code, e5m2 beyond 61440 -> infinity)."""
    for dt, top in ((torch.float8_e4m3fn, 16.0), (torch.float8_e5m2, 64.0)):
        vals = torch.tensor([0.0, 0.5, 1.0, 1.125, 1.5, 2.0, 3.5, 4.0, 6.0, 8.0, 11.0, top,
                             -1.0, -3.5, -8.0, -top])
        x = vals.repeat(4)[:64].to(dt)
        y = vals.flip(0).repeat(4)[:64].to(dt)
        a = torch.zeros(64, 128, dtype=dt)
        b = torch.zeros(64, 128, dtype=dt)
        a[:, 32:61] = x.view(64, 1).expand(64, 29)
        b[:, 32:61] = y.view(64, 1).expand(64, 29)
        c = torch.empty(64, 64, dtype=dt, device=DEV)
        ops.gemm(a.to(DEV), b.to(DEV), c, trans_b=True)
        exp = ref.gemm_fp8_ref(a, b)
        assert torch.equal(exp, 29 * x.float().view(64, 1) * y.float().view(1, 64))
        assert (exp.abs() > 480).any() and (exp == 464).any()
        e8 = exp.to(dt)
        got = c.cpu()
        nan = torch.isnan(e8.float())
        assert torch.equal(torch.isnan(got.float()), nan)
        assert torch.equal(got.view(torch.uint8)[~nan], e8.view(torch.uint8)[~nan])
