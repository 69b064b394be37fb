"""Golden fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py).

CPU: the oracle re-derives every stored input and elementwise output bit for bit (the fixtures
freeze it); outputs of float reductions (GEMM, attention, MLA, RMSNorm) match within one 16-bit rounding at
the output's scale, since torch's CPU reductions are split by thread count and a host with
another core count sums in another order.
GPU: each kernel family reproduces the stored outputs within the family's tolerance.
"""
import math
import os

import numpy as np
import pytest
import torch

from conftest import ROOT

GOLD = os.path.join(ROOT, "tests", "golden", "golden.npz")


def load():
    z = np.load(GOLD, allow_pickle=False)
    return {k: z[k] for k in z.files}


def t16(a, dt):
    return torch.from_numpy(a.view(np.int16).copy()).view(dt)


def t8(a):
    return torch.from_numpy(a.copy()).view(torch.float8_e4m3fn)


def test_fixtures_match_oracle():
    import sys
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_golden
    fresh = make_golden.cases()
    stored = load()
    assert set(fresh) == set(stored)
    f16, b16 = torch.float16, torch.bfloat16
    reductions = {"gemm_c": f16, "fa_o": b16, "mla_o": b16, "rmsnorm_y": f16}
    for k in stored:
        if k in reductions:
            # within one 16-bit rounding at the output's scale (an output that cancels to near
            # zero can differ by many of its own ulps)
            a = t16(fresh[k], reductions[k]).float()
            b = t16(stored[k], reductions[k]).float()
            eps = 2.0 ** -8 if reductions[k] == b16 else 2.0 ** -11
            tol = eps * float(b.abs().max())
            assert float((a - b).abs().max()) <= tol, (k, float((a - b).abs().max()), tol)
        else:
            assert np.array_equal(fresh[k], stored[k]), k


@pytest.mark.gpu
def test_kernels_match_fixtures():
    from tilelang.jit.adapter.mi355x import ops
    from tilelang.utils.tensor import torch_assert_close
    g = load()
    d = "cuda"
    f16, b16 = torch.float16, torch.bfloat16
    x, w = t16(g["rmsnorm_x"], f16).to(d), t16(g["rmsnorm_w"], f16).to(d)
    y = torch.empty_like(x)
    ops.rmsnorm(x, w, y, 1e-6)
    torch_assert_close(y.cpu(), t16(g["rmsnorm_y"], f16), atol=2e-3, rtol=2e-3)
    a, b = t16(g["gemm_a"], f16).to(d), t16(g["gemm_b"], f16).to(d)
    c = torch.empty(a.shape[0], b.shape[1], dtype=f16, device=d)
    ops.gemm(a, b, c)
    torch_assert_close(c.cpu(), t16(g["gemm_c"], f16), atol=1e-2, rtol=1e-2)
    q, k = t16(g["rope_q"], b16).to(d), t16(g["rope_k"], b16).to(d)
    cs, sn = t16(g["rope_cos"], b16).to(d), t16(g["rope_sin"], b16).to(d)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    ops.rope(q, cs, sn, qo, k, ko)
    torch_assert_close(qo.cpu(), t16(g["rope_q_out"], b16), atol=8e-3, rtol=8e-3)
    torch_assert_close(ko.cpu(), t16(g["rope_k_out"], b16), atol=8e-3, rtol=8e-3)
    ga, up = t16(g["swiglu_gate"], b16).to(d), t16(g["swiglu_up"], b16).to(d)
    o = torch.empty_like(ga)
    ops.swiglu(ga, up, o)
    torch_assert_close(o.cpu(), t16(g["swiglu_out"], b16), atol=8e-3, rtol=8e-3)
    fq, fk, fv = (t16(g[f"fa_{n}"], b16).to(d) for n in "qkv")
    fo = torch.empty_like(fq)
    ops.flash_attn_fwd(fq, fk, fv, fo, True, 1 / math.sqrt(64))
    torch_assert_close(fo.cpu(), t16(g["fa_o"], b16), atol=2e-2, rtol=2e-2)
    mq, kv = t16(g["mla_q"], b16).to(d), t8(g["mla_kv"]).to(d)
    bt = torch.from_numpy(g["mla_block_table"]).to(d)
    sl = torch.from_numpy(g["mla_seqlens"]).to(d)
    sc = torch.from_numpy(g["mla_kv_scale"]).to(d)
    B, H = mq.shape[:2]
    mo = torch.empty(B, H, 512, dtype=b16, device=d)
    ws = torch.empty(ops.mla_workspace_bytes(B, H, 512, 2), dtype=torch.uint8, device=d)
    ops.mla_decode(mq[..., :512], mq[..., 512:], kv[:, :512], kv[:, 512:], bt, sl, mo, ws, 16, 2,
                   1 / math.sqrt(192), sc)
    torch_assert_close(mo.cpu(), t16(g["mla_o"], b16), atol=2e-2, rtol=5e-2)
