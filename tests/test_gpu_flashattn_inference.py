"""GPU parity: the split-KV inference program examples/flash_attention/example_mha_inference.py
through ``tilelang.compile`` (flash_attn_split + combine, Q [batch, seq_q, heads, dim] over
K, V [batch, seq_kv, heads, dim]); it runs as one attention pass with seq_q != seq_kv.

Oracle: ref.mha_inference_ref (the example's ref_program, :206-213), pinned against SDPA and
the restated split + combine algorithm in test_oracle.py. Tolerance: the example's own
assert_allclose bound, rtol = atol = 1e-2 (:289), fp16 inputs.
"""
import pytest
import torch

import tilelang
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qkv(B, Sq, Skv, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, Sq, H, D, generator=g).half(),
            torch.randn(B, Skv, H, D, generator=g).half(),
            torch.randn(B, Skv, H, D, generator=g).half())


def test_example_config_gpu_convention():
    """The example's own call (:279-289): batch 1, 32 heads, 128 queries, 8192 keys, dim 128,
    block_M 128, block_N 64, 4 splits; out_idx=[5] (Q, K, V, glse, Output_partial in, Output
    out)."""
    B, H, Sq, Skv, D, ns = 1, 32, 128, 8192, 128, 4
    k = tilelang.compile(programs.mha_inference(B, H, Sq, Skv, D), out_idx=[5])
    assert k.plan.attrs["layout"] == "bshd_kv" and k.plan.attrs["num_split"] == ns
    q, kk, v = _qkv(B, Sq, Skv, H, D, 101)
    glse = torch.empty(B, H, ns, Sq, dtype=torch.float16, device=DEV)
    part = torch.empty(B, Sq, H, ns, D, dtype=torch.float16, device=DEV)
    out = k(q.to(DEV), kk.to(DEV), v.to(DEV), glse, part).cpu()
    torch_assert_close(out.float(), ref.mha_inference_ref(q, kk, v), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("B,H,Sq,Skv,D,bm,bn,ns", [(2, 8, 100, 1024, 64, 64, 64, 4),
                                                    (3, 4, 300, 768, 128, 128, 64, 2),
                                                    (1, 2, 1, 512, 128, 128, 64, 8)])
def test_other_shapes_tpu_convention(B, H, Sq, Skv, D, bm, bn, ns):
    k = tilelang.compile(programs.mha_inference(B, H, Sq, Skv, D, block_M=bm, block_N=bn,
                                                num_split=ns), out_idx=[5], target="tpu")
    q, kk, v = _qkv(B, Sq, Skv, H, D, 102 + Sq)
    glse = torch.zeros(B, H, ns, Sq, dtype=torch.float16)
    part = torch.zeros(B, Sq, H, ns, D, dtype=torch.float16)
    out = torch.zeros(B, Sq, H, D, dtype=torch.float16)
    assert k(q, kk, v, glse, part, out) == 0
    torch_assert_close(out.float(), ref.mha_inference_ref(q, kk, v), atol=1e-2, rtol=1e-2)
