"""GPU parity: the non-paged MLA decode programs through ``tilelang.compile``.

Programs: the TPU program tpu_demo/ppl/deepseek_mla/mla_decode.py:9-121 (T.ppl_* ops, natural
exp, Q / Output [batch, heads, 1, dim]) and the upstream examples/deepseek_mla/
example_mla_decode.py:10-227 (exp2 softmax, split and no-split forms). Both read a non-paged
cache KV [batch, seqlen_kv, 1, dim], which runs on the paged kernels through an identity block
table; shapes the matrix-core kernels do not take (the TPU demo's dim 32 + rope 4 over 8 heads)
run the generic decode kernel.
Oracle: ref.mla_decode_nopage_ref (ref_program, example_mla_decode.py:230-265).
Tolerance: the example's own assert_allclose bound, rtol = atol = 1e-2 (:327), fp16 inputs.
"""
import math

import pytest
import torch

import tilelang
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, H, S, dv, dpe, seed, q4=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, dv, generator=g).half()
    qpe = torch.randn(B, H, dpe, generator=g).half()
    kv = torch.randn(B, S, 1, dv, generator=g).half()
    kpe = torch.randn(B, S, 1, dpe, generator=g).half()
    if q4:
        q, qpe = q.unsqueeze(2), qpe.unsqueeze(2)
    return q, qpe, kv, kpe


def test_tpu_program_own_shape_tpu_convention():
    """The TPU demo's own call: flashattn(4, 8, 1, 512, 32, 4, 4, 4), CPU tensors, all params,
    output written in place, status 0."""
    B, H, S, dv, dpe = 4, 8, 512, 32, 4
    k = tilelang.compile(programs.mla_decode_tpu(B, H, S, dv, dpe, 4, 4), out_idx=-1,
                         target="tpu")
    assert k.plan.family == "mla" and not k.plan.attrs["paged"]
    q, qpe, kv, kpe = _inputs(B, H, S, dv, dpe, 81, q4=True)
    out = torch.zeros(B, H, 1, dv, dtype=torch.float16)
    assert k(q, qpe, kv, kpe, out) == 0
    torch_assert_close(out, ref.mla_decode_nopage_ref(q, qpe, kv, kpe), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("B,H,S", [(2, 8, 1), (3, 8, 100), (2, 24, 700)])
def test_tpu_program_generic_shapes(B, H, S):
    k = tilelang.compile(programs.mla_decode_tpu(B, H, S, 32, 4, 4, 4), out_idx=-1)
    q, qpe, kv, kpe = _inputs(B, H, S, 32, 4, 82 + S, q4=True)
    out = k(*(x.to(DEV) for x in (q, qpe, kv, kpe)))
    torch_assert_close(out.cpu(), ref.mla_decode_nopage_ref(q, qpe, kv, kpe), atol=1e-2,
                       rtol=1e-2)


def test_tpu_program_deepseek_shape():
    """The TPU program at DeepSeek-V3 dims (512 + 64, 128 heads), 8192 tokens: the fp16 KV runs
    on the matrix-core split kernel."""
    B, H, S, dv, dpe = 4, 128, 8192, 512, 64
    k = tilelang.compile(programs.mla_decode_tpu(B, H, S, dv, dpe, 64, 64), out_idx=-1)
    q, qpe, kv, kpe = _inputs(B, H, S, dv, dpe, 83, q4=True)
    out = k(*(x.to(DEV) for x in (q, qpe, kv, kpe))).cpu()
    torch_assert_close(out, ref.mla_decode_nopage_ref(q, qpe, kv, kpe), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("num_split", [1, 4])
def test_upstream_program_default_shape(num_split):
    """example_mla_decode.py's defaults: batch 128, 128 heads, 8192 tokens, 512 + 64 dims
    (main_no_split at num_split 1, main_split otherwise); the oracle checks 8 of the 128
    sequences, the first and last included."""
    B, H, S, dv, dpe = 128, 128, 8192, 512, 64
    k = tilelang.compile(programs.mla_decode_nopage(B, H, S, dv, dpe, num_split=num_split),
                         out_idx=[6])
    q, qpe, kv, kpe = _inputs(B, H, S, dv, dpe, 84)
    glse = torch.empty(B, H, num_split, dtype=torch.float16, device=DEV)
    opart = torch.empty(B, H, num_split, dv, dtype=torch.float16, device=DEV)
    out = k(q.to(DEV), qpe.to(DEV), kv.to(DEV), kpe.to(DEV), glse, opart).cpu()
    sel = [0, 17, 40, 63, 64, 99, 126, 127]
    exp = ref.mla_decode_nopage_ref(q[sel], qpe[sel], kv[sel], kpe[sel])
    torch_assert_close(out[sel], exp, atol=1e-2, rtol=1e-2)
    assert torch.isfinite(out.float()).all()


def test_upstream_program_config_batch():
    """B 64, 128 heads, 8192 tokens (the MLA config's batch and longest length) in bf16-free
    fp16 as the example declares; split form with 4 splits, every sequence checked."""
    B, H, S, dv, dpe = 64, 128, 8192, 512, 64
    k = tilelang.compile(programs.mla_decode_nopage(B, H, S, dv, dpe, num_split=4), out_idx=[6])
    q, qpe, kv, kpe = _inputs(B, H, S, dv, dpe, 85)
    glse = torch.empty(B, H, 4, dtype=torch.float16, device=DEV)
    opart = torch.empty(B, H, 4, dv, dtype=torch.float16, device=DEV)
    out = k(q.to(DEV), qpe.to(DEV), kv.to(DEV), kpe.to(DEV), glse, opart).cpu()
    torch_assert_close(out, ref.mla_decode_nopage_ref(q, qpe, kv, kpe), atol=1e-2, rtol=1e-2)
    # the split form's partials (example_mla_decode.py: split s covers tokens
    # [s S / 4, (s + 1) S / 4)), checked on sequences 0 and 63 through an identity block table
    sel = [0, 63]
    bt = torch.arange(2, dtype=torch.int32).view(2, 1)
    sl = torch.full((2,), S, dtype=torch.int32)
    _, (g_ref, p_ref) = ref.mla_split_combine_ref(
        q[sel], qpe[sel], kv[sel].reshape(2 * S, dv), kpe[sel].reshape(2 * S, dpe), bt, sl, S,
        1 / math.sqrt(dv + dpe), 4, block_n=64, store_dtype=torch.float16)
    torch_assert_close(glse[sel].cpu().float(), g_ref, atol=2e-2, rtol=0)
    torch_assert_close(opart[sel].cpu().float(), p_ref, atol=1e-2, rtol=1e-2)


def test_upstream_program_generic_heads():
    """16 heads (not a multiple of the matrix-core kernels' 64) run the generic kernel."""
    B, H, S, dv, dpe = 3, 16, 300, 512, 64
    k = tilelang.compile(programs.mla_decode_nopage(B, H, S, dv, dpe, block_H=16), out_idx=[6])
    q, qpe, kv, kpe = _inputs(B, H, S, dv, dpe, 86)
    g, op = torch.empty(B, H, 1, dtype=torch.float16), torch.empty(B, H, 1, dv, dtype=torch.float16)
    out = k(*(x.to(DEV) for x in (q, qpe, kv, kpe, g, op))).cpu()
    torch_assert_close(out, ref.mla_decode_nopage_ref(q, qpe, kv, kpe), atol=1e-2, rtol=1e-2)


def test_one_kernel_on_two_streams():
    """One compiled program on two streams whose work overlaps: each stream keeps its own
    workspace and identity table, so both results are the program's on their own inputs."""
    B, H, S, dv, dpe = 4, 128, 1024, 512, 64
    k = tilelang.compile(programs.mla_decode_nopage(B, H, S, dv, dpe, num_split=1), out_idx=[6])
    ins = [_inputs(B, H, S, dv, dpe, 130 + i) for i in range(2)]
    dev_ins = [tuple(x.to(DEV) for x in t) for t in ins]
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = []
    torch.cuda.synchronize()
    for _ in range(3):
        for s, (q, qpe, kv, kpe) in zip(streams, dev_ins):
            with torch.cuda.stream(s):
                glse = torch.empty(B, H, 1, dtype=torch.float16, device=DEV)
                opart = torch.empty(B, H, 1, dv, dtype=torch.float16, device=DEV)
                outs.append(k(q, qpe, kv, kpe, glse, opart))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        torch_assert_close(o.cpu(), ref.mla_decode_nopage_ref(*ins[i % 2]), atol=1e-2, rtol=1e-2)
