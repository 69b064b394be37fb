"""GPU parity of the allocation-free MLA entry point (tlm_mla_decode_noalloc) against
tlm_mla_decode with a caller workspace, both called through the C ABI.

The two entry points run the same kernels on the same inputs with the same workspace layout, so
the outputs must be bit-identical. Two calls in a row share the library's scratch array; the
second is smaller than the first (fewer sequences, fewer heads, shorter pages), so it runs on
scratch that still holds the first call's contents. A third call takes the split path (16-token
pages) through the same array.
"""
import ctypes

import pytest
import torch

from tilelang.jit.adapter.mi355x import lib, ops
from tilelang.testing import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(t, a, out):
    q, kv = t["q"], t["kv"]
    B, Hq = q.shape[0], q.shape[1]
    return [q.data_ptr(), q[..., 512:].data_ptr(), q.stride(1), q.stride(1), kv.data_ptr(),
            kv[:, 512:].data_ptr(), kv.stride(0), kv.stride(0), kv.shape[0],
            t["block_table"].data_ptr(), t["seqlens"].data_ptr(), out.data_ptr()], \
        [B, Hq, 512, 64, a["page"], t["block_table"].shape[1]]


def _both(w, num_split):
    a = w.attrs
    t = {k: v.to(DEV) for k, v in w.tensors.items()}
    B, Hq = t["q"].shape[0], t["q"].shape[1]
    L = lib.load()
    lib.ensure_device(torch.cuda.current_device())
    stream = torch.cuda.current_stream().cuda_stream
    tail = [num_split, a["sm_scale"], t["kv_scale"].data_ptr(), lib.BF16, lib.F8E4M3, lib.BF16,
            stream]
    out_ws = torch.full((B, Hq, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    nbytes = L.tlm_mla_workspace_bytes(B, Hq, 512, num_split)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    head, sizes = _args(t, a, out_ws)
    lib.check("tlm_mla_decode", L.tlm_mla_decode(*head, ws.data_ptr(), nbytes, *sizes, *tail))
    out_na = torch.full((B, Hq, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    head, sizes = _args(t, a, out_na)
    print(f"[no_alloc] B={B} Hq={Hq} page={a['page']} splits={num_split}", flush=True)
    lib.check("tlm_mla_decode_noalloc", L.tlm_mla_decode_noalloc(*head, *sizes, *tail))
    torch.cuda.synchronize()
    return out_ws.cpu(), out_na.cpu()


def test_noalloc_matches_workspace_entry_two_calls():
    first = workloads.mla(B=24, Hq=128, max_pages=40, min_len=500, max_len=2560, seed=91)
    ref1, got1 = _both(first, 4)
    assert not torch.isnan(got1).any()
    assert torch.equal(ref1, got1)
    second = workloads.mla(B=5, Hq=64, max_pages=12, min_len=1, max_len=768, seed=92)
    ref2, got2 = _both(second, 2)
    assert not torch.isnan(got2).any()
    assert torch.equal(ref2, got2)


def test_noalloc_split_path():
    w = workloads.mla(B=6, Hq=64, page=16, max_pages=40, min_len=50, max_len=640, seed=93)
    ref, got = _both(w, 3)
    assert not torch.isnan(got).any()
    assert torch.equal(ref, got)


def test_noalloc_rejects_oversized_request():
    w = workloads.mla(B=2, Hq=64, max_pages=2, min_len=64, max_len=128, seed=94)
    a = w.attrs
    t = {k: v.to(DEV) for k, v in w.tensors.items()}
    out = torch.empty(2, 64, 512, dtype=torch.bfloat16, device=DEV)
    head, sizes = _args(t, a, out)
    sizes[0] = 1 << 20  # a batch far beyond the scratch
    L = lib.load()
    rc = L.tlm_mla_decode_noalloc(*head, *sizes, 64, a["sm_scale"], t["kv_scale"].data_ptr(),
                                  lib.BF16, lib.F8E4M3, lib.BF16,
                                  torch.cuda.current_stream().cuda_stream)
    assert rc == -4 and b"scratch" in L.tlm_last_error()
