"""GPU parity: paged KV-cache append with FP8 quantisation (tlm_kv_append_fp8), bit-exact
against oracle.ref.kv_append_fp8_ref (page addressing example_mla_decode_paged.py:62-63; codes =
torch's RNE e4m3 cast after clamping to +-448, pinned by a brute-force nearest-even check in
tests/test_oracle.py). Bytes are compared exactly; NaN inputs are compared as NaN codes."""
import numpy as np
import pytest
import torch

from tilelang.jit.adapter.mi355x import ops
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(x, start, count, bt, pool_u8, page, scale):
    kv = torch.from_numpy(pool_u8.copy()).to(DEV).view(torch.float8_e4m3fn)
    ops.kv_append_fp8(x.to(DEV), torch.as_tensor(start, dtype=torch.int32).to(DEV),
                      torch.as_tensor(count, dtype=torch.int32).to(DEV),
                      torch.as_tensor(bt, dtype=torch.int32).to(DEV), kv, page,
                      torch.tensor([scale], dtype=torch.float32, device=DEV))
    torch.cuda.synchronize()
    return kv.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_random_appends_bit_exact(dtype):
    g = torch.Generator().manual_seed(41)
    B, T, D, page, pages = 6, 70, 576, 64, 5
    x = (torch.randn(B, T, D, generator=g) * 3).to(dtype)
    bt = torch.randperm(B * pages, generator=g).view(B, pages).to(torch.int32).numpy()
    start = np.array([0, 5, 63, 64, 250, 100], dtype=np.int32)   # page crossings, table end
    count = np.array([70, 0, 2, 64, 70, 33], dtype=np.int32)
    pool = np.full((B * pages * page + 7, D), 0xA5, dtype=np.uint8)  # untouched rows stay 0xA5
    scale = float(x.float().abs().max()) / 448.0
    got = _run(x, start, count, bt, pool, page, scale)
    exp = ref.kv_append_fp8_ref(x, start, count, bt, pool, page, scale)
    assert np.array_equal(got, exp)


def test_every_bf16_value_bit_exact():
    """All 65536 bf16 bit patterns through the quantiser (scale 1): finite values saturate at
    +-448, NaN stays NaN; everything else equals torch's RNE cast."""
    allbits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = allbits.view(1, 65536 // 64, 64)
    page, T = 64, x.shape[1]
    bt = np.arange(16, dtype=np.int32).reshape(1, 16)
    pool = np.zeros((16 * page, 64), dtype=np.uint8)
    got = _run(x, np.array([0]), np.array([T]), bt, pool, page, 1.0)
    exp = ref.kv_append_fp8_ref(x, np.array([0]), np.array([T]), bt, pool, page, 1.0)
    table = ref.fp8_e4m3fn_table()
    gnan, enan = np.isnan(table[got]), np.isnan(table[exp])
    assert np.array_equal(gnan, enan)
    assert np.array_equal(got[~gnan], exp[~enan])


def test_corrupt_table_entries_write_nothing():
    g = torch.Generator().manual_seed(42)
    B, T, D, page = 2, 10, 64, 8
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    bt = np.array([[1, -5], [1 << 20, 0]], dtype=np.int32)
    pool = np.full((4 * page, D), 0x11, dtype=np.uint8)
    got = _run(x, np.array([4, 0]), np.array([10, 10]), bt, pool, page, 0.02)
    exp = ref.kv_append_fp8_ref(x, np.array([4, 0]), np.array([10, 10]), bt, pool, page, 0.02)
    assert np.array_equal(got, exp)
    # written: sequence 0 positions 4..7 (page 1, rows 12..15; positions 8..13 hit page -5) and
    # sequence 1 positions 8, 9 (page 0, rows 0, 1; positions 0..7 hit page 2^20)
    changed = np.flatnonzero((got != 0x11).any(axis=1))
    assert changed.tolist() == [0, 1, 12, 13, 14, 15]


def test_cache_built_by_append_decodes_like_the_config_cache():
    """Fill an empty paged pool token by token (decode-style) from the MLA config's latent rows:
    the result equals the config's own fp8 cache, so the decode reads identical bytes."""
    from tilelang.testing import workloads
    w = workloads.mla(B=4, max_pages=6, min_len=100, max_len=384, seed=43)
    T_, a = w.tensors, w.attrs
    page, pages = a["page"], a["max_pages"]
    bt, sl = T_["block_table"], T_["seqlens"]
    scale = float(T_["kv_scale"])
    kv_ref = T_["kv"].view(torch.uint8).numpy()
    # latent rows that quantise exactly to the config's codes: their dequantised values
    lat = (T_["kv"].float() * scale).to(torch.bfloat16)
    B, L = bt.shape[0], int(sl.max())
    x = torch.zeros(B, L, 576, dtype=torch.bfloat16)
    for b in range(B):
        rows = ref.paged_rows(bt, int(sl[b]), b, page)
        x[b, :int(sl[b])] = lat[rows]
    pool = np.zeros_like(kv_ref)
    got = _run(x, np.zeros(B, np.int32), sl.numpy(), bt.numpy(), pool, page, scale)
    exp = ref.kv_append_fp8_ref(x, np.zeros(B, np.int32), sl.numpy(), bt.numpy(), pool, page,
                                scale)
    assert np.array_equal(got, exp)
    for b in range(B):
        rows = ref.paged_rows(bt, int(sl[b]), b, page).numpy()
        assert np.array_equal(got[rows], kv_ref[rows])


def test_random_scales_bit_exact():
    """x / scale is correctly rounded for any positive normal scale (the kernel refines x * (1/s)
    instead of dividing): random scales and inputs, including tiny, zero and huge values."""
    g = torch.Generator().manual_seed(44)
    page = 64
    for trial in range(6):
        scale = float(torch.exp(torch.randn(1, generator=g) * 8))
        x = torch.randn(1, 4096, 64, generator=g) * float(torch.exp(torch.randn(1, generator=g) * 6))
        x[0, :8] = torch.tensor([0.0, -0.0, 1e-35, -1e-38, 3e38, float("inf"), float("-inf"),
                                 float("nan")]).view(8, 1)
        x = x.to(torch.bfloat16)
        bt = np.arange(64, dtype=np.int32).reshape(1, 64)
        pool = np.zeros((64 * page, 64), dtype=np.uint8)
        got = _run(x, np.array([0]), np.array([4096]), bt, pool, page, scale)
        exp = ref.kv_append_fp8_ref(x, np.array([0]), np.array([4096]), bt, pool, page, scale)
        table = ref.fp8_e4m3fn_table()
        gn, en = np.isnan(table[got]), np.isnan(table[exp])
        assert np.array_equal(gn, en), trial
        assert np.array_equal(got[~gn], exp[~en]), trial


@pytest.mark.parametrize("D,width", [(72, 72), (64, 72), (512, 576)])
def test_column_slices_and_8_wide_rows(D, width):
    """kv given as the first D columns of a wider pool (the latent part of a fused [rows, 576]
    cache) and row strides that are not multiples of 16 bytes (8-element kernel variant); the
    columns beyond D stay untouched."""
    g = torch.Generator().manual_seed(45)
    B, T, page, pages = 3, 50, 16, 4
    x = (torch.randn(B, T, D, generator=g) * 2).to(torch.bfloat16)
    bt = torch.randperm(B * pages, generator=g).view(B, pages).to(torch.int32).numpy()
    start = np.array([0, 13, 30], dtype=np.int32)
    count = np.array([50, 20, 34], dtype=np.int32)
    pool = np.full((B * pages * page, width), 0x5A, dtype=np.uint8)
    full = torch.from_numpy(pool.copy()).to(DEV).view(torch.float8_e4m3fn)
    ops.kv_append_fp8(x.to(DEV), torch.as_tensor(start).to(DEV), torch.as_tensor(count).to(DEV),
                      torch.as_tensor(bt).to(DEV), full[:, :D], page,
                      torch.tensor([0.01], dtype=torch.float32, device=DEV))
    torch.cuda.synchronize()
    got = full.view(torch.uint8).cpu().numpy()
    exp = pool.copy()
    exp[:, :D] = ref.kv_append_fp8_ref(x, start, count, bt, pool[:, :D], page, 0.01)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("scale", [2.0 ** -126, 2.0 ** -100, 2.0 ** -90, 2.0 ** -89.5,
                                   2.0 ** 89.5, 2.0 ** 90, 2.0 ** 100, 3e38])
def test_extreme_scales_every_bf16_value(scale):
    """Every bf16 bit pattern at scales on both sides of the kernel's fast-path window
    [2^-90, 2^90] (outside it the kernel divides per element): bf16 subnormals against the
    smallest normal scale, quotients that overflow fp32, exact signed zeros."""
    allbits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = allbits.view(1, 65536 // 64, 64)
    page, T = 64, x.shape[1]
    bt = np.arange(16, dtype=np.int32).reshape(1, 16)
    pool = np.zeros((16 * page, 64), dtype=np.uint8)
    got = _run(x, np.array([0]), np.array([T]), bt, pool, page, scale)
    exp = ref.kv_append_fp8_ref(x, np.array([0]), np.array([T]), bt, pool, page, scale)
    table = ref.fp8_e4m3fn_table()
    gnan, enan = np.isnan(table[got]), np.isnan(table[exp])
    assert np.array_equal(gnan, enan)
    assert np.array_equal(got[~gnan], exp[~enan])
