"""GPU parity: the split-KV inference program examples/flash_attention/example_mha_inference.py
through ``tilelang.compile`` (flash_attn_split + combine, Q [batch, seq_q, heads, dim] over
K, V [batch, seq_kv, heads, dim]). The kernels write the program's partials as the program does:
glse [batch, heads, num_split, seq_q] (each split's log2 sum-exp) and Output_partial
[batch, seq_q, heads, num_split, dim] (each split's normalised output), rounded to the program's
dtype, and Output is the combine of those stored values.

Oracles: ref.mha_inference_ref (the example's ref_program, :206-213) for Output, and
ref.mha_split_combine_ref (flash_split_ref + reduce_ref, :216-275, pinned in test_oracle.py)
for glse, Output_partial and the combine of the stored values. Tolerance: the example's own
assert_allclose bound, rtol = atol = 1e-2 (:289), fp16 inputs; glse within 2e-2 (one fp16 ulp
of a log2 sum-exp near 16 is 2^-7).
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
    _check_partials(q, kk, v, ns, 64, glse.cpu(), part.cpu(), out)


def _check_partials(q, kk, v, ns, bn, glse, part, out):
    """The written glse / Output_partial against the restated flash_split_ref, and Output
    against the restated reduce_ref of the stored values."""
    comb, (g_ref, p_ref) = ref.mha_split_combine_ref(q, kk, v, ns, bn, store_dtype=q.dtype)
    torch_assert_close(glse.float(), g_ref, atol=2e-2, rtol=0)
    torch_assert_close(part.float(), p_ref, atol=1e-2, rtol=1e-2)
    torch_assert_close(out.float(), comb, atol=1e-2, rtol=1e-2)


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
    # host tensors: only the result (out_idx) is copied back, as the reference's TPU call copies
    # back result_idx alone (jit/adapter/cython/adapter.py:233-241)
    assert not glse.any() and not part.any()
    # device tensors are written in place, the partials included
    gd, pd, od = (x.to(DEV) for x in (glse, part, out))
    assert k(q.to(DEV), kk.to(DEV), v.to(DEV), gd, pd, od) == 0
    _check_partials(q, kk, v, ns, bn, gd.cpu(), pd.cpu(), od.cpu())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_partials_split_and_part_boundaries(dtype):
    """Keys whose scores rise by a large step inside one split: the split's lse and partial
    follow the step, the combine weights the splits by them. 2 heads of dim 128 over 4096 keys
    in 4 splits, 300 queries (two query tiles, the second partial)."""
    from tilelang.jit.adapter.mi355x import ops
    B, H, Sq, Skv, D, ns = 1, 2, 300, 4096, 128, 4
    g = torch.Generator().manual_seed(111)
    q = torch.randn(B, Sq, H, D, generator=g).to(dtype)
    kk = torch.randn(B, Skv, H, D, generator=g)
    kk[:, 1700:1800] += 0.5  # inside split 1
    kk = kk.to(dtype)
    v = torch.randn(B, Skv, H, D, generator=g).to(dtype)
    glse = torch.empty(B, H, ns, Sq, dtype=dtype, device=DEV)
    part = torch.empty(B, Sq, H, ns, D, dtype=dtype, device=DEV)
    out = torch.empty(B, Sq, H, D, dtype=dtype, device=DEV)
    ws = torch.empty(ops.flash_attn_splitkv_workspace_bytes(B, Sq, Skv, H, D, ns),
                     dtype=torch.uint8, device=DEV)
    ops.flash_attn_splitkv_fwd(q.to(DEV), kk.to(DEV), v.to(DEV), glse, part, out, ns,
                               D ** -0.5, ws)
    torch.cuda.synchronize()
    comb, (g_ref, p_ref) = ref.mha_split_combine_ref(q, kk, v, ns, 64, store_dtype=dtype)
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    # one ulp of a log2 sum-exp in [16, 32): 2^-6 in fp16, 2^-3 in bf16
    torch_assert_close(glse.cpu().float(), g_ref, atol=0.13 if dtype == torch.bfloat16 else 2e-2,
                       rtol=0)
    torch_assert_close(part.cpu().float(), p_ref, atol=tol, rtol=tol)
    torch_assert_close(out.cpu().float(), comb, atol=tol, rtol=tol)
    torch_assert_close(out.cpu().float(), ref.mha_inference_ref(q, kk, v), atol=tol, rtol=tol)


@pytest.mark.parametrize("D", [128, 64])
def test_grouped_kv_heads_equal_repeated_heads(D):
    """The C ABI's split-KV call with grouped K/V heads (query head h reads K/V head
    h // (H / H_kv), example_gqa_fwd_bshd.py:92-100) equals the call on K/V repeated per group,
    bit for bit: glse, Output_partial and Output (D 128 on the tiled kernel, D 64 on the
    per-query kernel)."""
    from tilelang.jit.adapter.mi355x import ops
    B, H, Hkv, Sq, Skv, ns = 2, 8, 2, 130, 2048, 4
    g = torch.Generator().manual_seed(113 + D)
    q = torch.randn(B, Sq, H, D, generator=g).half().to(DEV)
    kk = torch.randn(B, Skv, Hkv, D, generator=g).half().to(DEV)
    v = torch.randn(B, Skv, Hkv, D, generator=g).half().to(DEV)
    rep = lambda t: t.repeat_interleave(H // Hkv, dim=2).contiguous()
    outs = []
    for k_, v_ in ((kk, v), (rep(kk), rep(v))):
        glse = torch.full((B, H, ns, Sq), float("nan"), dtype=torch.half, device=DEV)
        part = torch.full((B, Sq, H, ns, D), float("nan"), dtype=torch.half, device=DEV)
        out = torch.full((B, Sq, H, D), float("nan"), dtype=torch.half, device=DEV)
        ws = torch.empty(ops.flash_attn_splitkv_workspace_bytes(B, Sq, Skv, H, D, ns),
                         dtype=torch.uint8, device=DEV)
        ops.flash_attn_splitkv_fwd(q, k_, v_, glse, part, out, ns, D ** -0.5, ws)
        outs.append((glse.cpu(), part.cpu(), out.cpu()))
    for a, b in zip(*outs):
        assert not a.isnan().any()
        assert torch.equal(a, b)
    torch_assert_close(outs[0][2].float(),
                       ref.mha_inference_ref(q.cpu(), rep(kk).cpu(), rep(v).cpu()),
                       atol=1e-2, rtol=1e-2)


def test_one_kernel_on_two_streams():
    """One compiled program called on two streams whose work overlaps: each stream has its own
    workspace, so both results equal the program's on their own inputs."""
    B, H, Sq, Skv, D, ns = 1, 8, 64, 2048, 128, 4
    k = tilelang.compile(programs.mha_inference(B, H, Sq, Skv, D), out_idx=[5])
    ins = [_qkv(B, Sq, Skv, H, D, 120 + i) for i in range(2)]
    dev_ins = [tuple(x.to(DEV) for x in qkv) for qkv in ins]
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = []
    torch.cuda.synchronize()
    for _ in range(3):
        for s, (q, kk, v) in zip(streams, dev_ins):
            with torch.cuda.stream(s):
                glse = torch.empty(B, H, ns, Sq, dtype=torch.float16, device=DEV)
                part = torch.empty(B, Sq, H, ns, D, dtype=torch.float16, device=DEV)
                outs.append(k(q, kk, v, glse, part))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        q, kk, v = ins[i % 2]
        torch_assert_close(o.cpu().float(), ref.mha_inference_ref(q, kk, v), atol=1e-2,
                           rtol=1e-2)
