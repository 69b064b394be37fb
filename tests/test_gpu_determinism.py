"""Determinism reruns (the reference's ``Profiler.assert_consistent`` pattern): every kernel family,
run several times on the same inputs, must give bit-identical outputs. A race between waves (an
LDS stage reused too early, a missing wait) shows up as run-to-run differences. Families whose
inputs must be valid indices (cu_seqlens, block tables, gather indices) get explicit inputs; the
rest use the profiler's random supply.
"""
import itertools

import pytest
import torch

import tilelang
from tilelang.jit.adapter.mi355x import ops
from tilelang.testing import programs, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPEAT = 4


@pytest.mark.parametrize("name,prog,out_idx", [
    ("gemm_rowmajor_b", lambda: programs.matmul(512, 768, 1024, 256, 256, 64), -1),
    ("gemm_bt_bf16", lambda: programs.matmul(300, 520, 256, 256, 256, 64, "bfloat16",
                                             "bfloat16", trans_b=True), -1),
    ("gemm_skinny", lambda: programs.matmul(16, 4096, 1024, 16, 64, 64), -1),
    ("gemm_fp8", lambda: programs.matmul_fp8(512, 512, 1024, 128, 128, 64, "e4m3_float8",
                                             two_acc=True), -1),
    ("flashattn_causal_paired", lambda: programs.flashattn(2, 4, 1100, 128, True), -1),
    ("flashattn_full", lambda: programs.flashattn(1, 4, 700, 128, False), -1),
    ("flashattn_gqa_causal", lambda: programs.flashattn_gqa(1, 8, 1024, 128, True, 4), [3]),
    ("flashattn_d64", lambda: programs.flashattn(1, 2, 600, 64, True), -1),
    ("flashattn_bhsd", lambda: programs.flashattn_bhsd(2, 4, 700, 900, 128, False), [3]),
    ("rmsnorm_splitk", lambda: programs.rms_norm_splitk(512, 512, 32, 32), -1),
    ("rope", lambda: programs.rope(64, 16, 256, 128), -1),
    ("swiglu", lambda: programs.swi_glu(32, 32, 256, 1024), -1),
    ("sigmoid", lambda: programs.sigmoid(32, 32, 256, 256), -1),
    ("row_sum", lambda: programs.row_reduce(256, 1000, 32, 1000, "sum"), -1),
])
def test_profiler_assert_consistent(name, prog, out_idx):
    k = tilelang.compile(prog(), out_idx=out_idx, target="mi355x")
    k.get_profiler().assert_consistent(repeat=REPEAT)


def _same(runs):
    ref = runs[0]
    for r in runs[1:]:
        assert torch.equal(r.view(torch.uint8), ref.view(torch.uint8))


def test_flashattn_varlen_consistent():
    lens = [300, 1, 700, 513, 64]
    cu = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.int32, device=DEV)
    T, H, D = int(cu[-1]), 8, 128
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(T, H, D, generator=g).half().to(DEV) for _ in range(3))
    kern = tilelang.compile(programs.flashattn_varlen(len(lens), T, T, H, D), out_idx=-1)
    _same([kern(q, k, v, cu, cu, max(lens)).clone() for _ in range(REPEAT)])
    for causal in (False, True):
        runs = []
        for _ in range(REPEAT):
            o = torch.empty_like(q)
            ops.flash_attn_varlen_fwd(q, k, v, cu, cu, max(lens), o, causal, 0.09)
            runs.append(o)
        _same(runs)


def test_mla_fp8_consistent():
    w = workloads.mla(B=6, max_pages=16, min_len=100, max_len=1000, seed=7)
    t = {n: x.to(DEV) for n, x in w.tensors.items()}
    a = w.attrs
    q, kv = t["q"], t["kv"]
    B, Hq = q.shape[0], q.shape[1]
    runs = []
    for num_split in (1, 3):
        ws = torch.empty(ops.mla_workspace_bytes(B, Hq, 512, num_split), dtype=torch.uint8,
                         device=DEV)
        outs = []
        for _ in range(REPEAT):
            out = torch.empty(B, Hq, 512, dtype=torch.bfloat16, device=DEV)
            ops.mla_decode(q[..., :512], q[..., 512:], kv[:, :512], kv[:, 512:],
                           t["block_table"], t["seqlens"], out, ws, a["page"], num_split,
                           a["sm_scale"], t["kv_scale"])
            outs.append(out)
        _same(outs)
        runs.append(outs[0])


def test_index_ops_consistent():
    g = torch.Generator().manual_seed(9)
    param = torch.randn(4000, 96, generator=g).to(DEV)
    idx = torch.randint(0, 4000, (2500,), generator=g).to(torch.int32).to(DEV)
    _same([ops.gather_rows(param, idx, torch.empty(2500, 96, device=DEV)) for _ in range(3)])
    src = (torch.randint(0, 40, (5000,), generator=g).float() / 4).to(DEV)  # many ties
    vals, idxs = [], []
    for _ in range(3):
        v = torch.empty(5000, device=DEV)
        i = torch.empty(5000, dtype=torch.int32, device=DEV)
        ops.topk(src, 10, True, v, i)
        vals.append(v)
        idxs.append(i)
    _same(vals)
    _same(idxs)


def test_kv_append_consistent():
    B, T, D, page, max_pages = 4, 96, 576, 64, 8
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, T, D, generator=g).bfloat16().to(DEV)
    start = torch.tensor([0, 70, 5, 300], dtype=torch.int32, device=DEV)
    count = torch.tensor([96, 50, 0, 96], dtype=torch.int32, device=DEV)
    table = torch.randperm(B * max_pages, generator=g).view(B, max_pages).to(torch.int32)
    table = table.to(DEV)
    scale = torch.tensor([0.02], device=DEV)
    runs = []
    for _ in range(3):
        kv = torch.zeros(B * max_pages * page, D, dtype=torch.float8_e4m3fn, device=DEV)
        ops.kv_append_fp8(x, start, count, table, kv, page, scale)
        runs.append(kv)
    _same(runs)
