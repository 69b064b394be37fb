"""GPU parity: the generic MLA decode kernel (`mla_generic_kernel`, one workgroup per (sequence,
head)) on the requests that the matrix-core kernels do not take.

Cases: fp8 KV with 16 heads (kv_scale applied to the scores and to the output), a random block
table whose pages lie outside the pool for part of a sequence, and 64-head dv 512 / dpe 64
inputs whose Q rows start at an odd element offset (the fast kernels need 16-byte aligned rows,
so the request falls back to this kernel).
Oracle: ref.mla_decode_ref (restated run_torch_mla, examples/deepseek_mla/
example_mla_decode_paged.py:259-308) on the dequantised cache; a page outside the pool is a page
of zero rows. The kernel rounds P to Q's 16-bit dtype before PV as the programs' P tiles are, so
the bound is the 16-bit one: atol 2e-2, rtol 5e-2, relative RMS below 1%.
"""
import math

import pytest
import torch

from tilelang.jit.adapter.mi355x import ops
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
PAGE = 64


def _rel_rms(a, b):
    a, b = a.float(), b.float()
    return float(((a - b).pow(2).mean() / b.pow(2).mean().clamp_min(1e-30)).sqrt())


def _inputs(B, Hq, max_pages, kv_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(PAGE + 1, max_pages * PAGE + 1, (B,), generator=g).to(torch.int32)
    table = torch.randperm(B * max_pages, generator=g).view(B, max_pages).to(torch.int32)
    latent = torch.randn(B * max_pages * PAGE, 576, generator=g)
    if kv_dtype == torch.float8_e4m3fn:
        scale = float(latent.abs().max()) / 448.0
        kv = (latent / scale).to(torch.float8_e4m3fn)
    else:
        scale = 1.0
        kv = latent.to(kv_dtype)
    q = torch.randn(B, Hq, 576, generator=g).to(torch.bfloat16)
    return q, kv, table, lens, scale


def _decode(q, kv, table, lens, scale, kv_scale_tensor):
    B, Hq = q.shape[0], q.shape[1]
    out = torch.empty(B, Hq, 512, dtype=torch.bfloat16, device=DEV)
    ws = torch.empty(max(ops.mla_workspace_bytes(B, Hq, 512, 1), 16), dtype=torch.uint8,
                     device=DEV)
    kvd = kv.to(DEV)
    ops.mla_decode(q[..., :512], q[..., 512:], kvd[:, :512], kvd[:, 512:], table.to(DEV),
                   lens.to(DEV), out, ws, PAGE, 1, 1 / math.sqrt(576), kv_scale_tensor)
    torch.cuda.synchronize()
    return out.cpu()


def _check(got, exp):
    torch_assert_close(got, exp, atol=2e-2, rtol=5e-2)
    assert _rel_rms(got, exp) < 0.01


def test_fp8_kv_16_heads():
    q, kv, table, lens, scale = _inputs(3, 16, 6, torch.float8_e4m3fn, 91)
    got = _decode(q.to(DEV), kv, table, lens, scale,
                  torch.tensor([scale], dtype=torch.float32, device=DEV))
    exp = ref.mla_decode_ref(q[..., :512], q[..., 512:], kv[:, :512], kv[:, 512:], table, lens,
                             PAGE, 1 / math.sqrt(576), scale)
    _check(got, exp)


def test_pages_outside_the_pool_with_16_heads():
    """Table entries past the pool (below the sequence length) read as zero rows: the result
    equals a pool extended by one all-zero page that those entries point to."""
    q, kv, table, lens, _ = _inputs(3, 16, 6, torch.bfloat16, 92)
    lens = torch.tensor([6 * PAGE, 5 * PAGE - 7, 3 * PAGE + 1], dtype=torch.int32)
    bt = table.clone()
    bt[0, 1] = 1_000_000
    bt[1, 4] = bt.numel() + 3  # just past the pool
    bt[2, 0] = 2 ** 30
    got = _decode(q.to(DEV), kv, bt, lens, 1.0, None)
    zero_page = kv.shape[0] // PAGE
    kv2 = torch.cat([kv, torch.zeros(PAGE, 576, dtype=kv.dtype)])
    bt2 = bt.clone()
    bt2[0, 1] = bt2[1, 4] = bt2[2, 0] = zero_page
    exp = ref.mla_decode_ref(q[..., :512], q[..., 512:], kv2[:, :512], kv2[:, 512:], bt2, lens,
                             PAGE, 1 / math.sqrt(576), 1.0)
    _check(got, exp)


def test_odd_offset_q_rows_fall_back():
    """64 heads at dv 512 / dpe 64 take the matrix-core kernels only with 16-byte aligned Q rows;
    Q rows starting at an odd element offset run the generic kernel with the same result."""
    B, Hq = 2, 64
    q, kv, table, lens, scale = _inputs(B, Hq, 5, torch.float8_e4m3fn, 93)
    flat = torch.zeros(B * Hq * 576 + 1, dtype=torch.bfloat16, device=DEV)
    qv = flat[1:].view(B, Hq, 576)
    qv.copy_(q.to(DEV))
    assert qv.data_ptr() % 16 != 0
    kvs = torch.tensor([scale], dtype=torch.float32, device=DEV)
    got = _decode(qv, kv, table, lens, scale, kvs)
    exp = ref.mla_decode_ref(q[..., :512], q[..., 512:], kv[:, :512], kv[:, 512:], table, lens,
                             PAGE, 1 / math.sqrt(576), scale)
    _check(got, exp)
    # the aligned copy takes the fp8 matrix-core kernel; both stay within the FP8 bound
    aligned = _decode(q.to(DEV), kv, table, lens, scale, kvs)
    torch_assert_close(aligned, exp, atol=2e-2, rtol=5e-2)
