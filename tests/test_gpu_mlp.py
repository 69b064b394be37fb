"""GPU parity: the DeepSeek-V3 MLP program tpu_demo/ppl/mlp/mlp_bf16.py through
``tilelang.compile`` with whole hidden / intermediate blocks (the blocking under which the
program is the MLP), run as gate / up gemms, SwiGLU and the down gemm.

Oracle: ref.mlp_ref (pinned against the gemm / SwiGLU oracles and scalar loops). Tolerance: the
gemm tests' atol = rtol = 1e-2 (tpu_test_matmul_fp16.py:56) on the output, where a one-ulp
difference of a bf16 gate / up element (summation order) can move an output element by more
than 1e-2 relative in rare cases (at most 0.5% of the elements), and relative RMS error <= 1%.
"""
import pytest
import torch

import tilelang
from tilelang.testing import programs
from tilelang.utils.tensor import torch_assert_close
from oracle import ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weights(M, Hd, I, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, Hd, generator=g).to(dtype)
    wg = (torch.randn(I, Hd, generator=g) * Hd ** -0.5).to(dtype)
    wu = (torch.randn(I, Hd, generator=g) * Hd ** -0.5).to(dtype)
    wd = (torch.randn(Hd, I, generator=g) * I ** -0.5).to(dtype)
    return x, wg, wu, wd


def _check(out, exp):
    out, exp = out.float(), exp.float()
    torch_assert_close(out, exp, atol=1e-2, rtol=1e-2, max_mismatched_ratio=0.005)
    assert ((out - exp).pow(2).mean() / exp.pow(2).mean()).sqrt() < 0.01


def test_demo_shape_whole_blocks_tpu_convention():
    """The demo's sizes (batch_seq = hidden = intermediate = 16) with 16-wide blocks; TPU
    convention: CPU tensors, all parameters, output (parameter 0) written in place."""
    k = tilelang.compile(programs.deepseek_mlp(16, 16, 16, 16, 16, 16), out_idx=[0],
                         target="tpu")
    assert k.plan.family == "mlp"
    x, wg, wu, wd = _weights(16, 16, 16, 111)
    out = torch.zeros(16, 16, dtype=torch.bfloat16)
    assert k(out, x, wg, wu, wd) == 0
    _check(out, ref.mlp_ref(x, wg, wu, wd))


@pytest.mark.parametrize("M,Hd,I,dtype", [(512, 7168, 2048, torch.bfloat16),
                                          (96, 256, 768, torch.bfloat16),
                                          (64, 512, 1024, torch.float16)])
def test_deepseek_shapes(M, Hd, I, dtype):
    """DeepSeek-V3 MoE expert dims (hidden 7168, intermediate 2048) and smaller ragged ones."""
    dt = "bfloat16" if dtype == torch.bfloat16 else "float16"
    k = tilelang.compile(programs.deepseek_mlp(min(M, 64), Hd, I, M, Hd, I, dtype=dt),
                         out_idx=[0])
    x, wg, wu, wd = _weights(M, Hd, I, 112 + M, dtype)
    out = k(x.to(DEV), wg.to(DEV), wu.to(DEV), wd.to(DEV)).cpu()
    _check(out, ref.mlp_ref(x, wg, wu, wd))


@pytest.mark.parametrize("M,Hd,I", [(16, 16, 16), (96, 512, 1024)])
def test_fp32_program(M, Hd, I):
    """tpu_demo/ppl/mlp/mlp_fp32.py with whole blocks: fp32 parameters and output, bf16 gemm
    tiles (the demo's own 16 x 16 x 16 and a larger shape)."""
    k = tilelang.compile(programs.deepseek_mlp_fp32(min(M, 64), Hd, I, M, Hd, I), out_idx=[0])
    x, wg, wu, wd = _weights(M, Hd, I, 113 + M, torch.float32)
    out = k(x.to(DEV), wg.to(DEV), wu.to(DEV), wd.to(DEV)).cpu()
    assert out.dtype == torch.float32
    _check(out, ref.mlp_ref(x, wg, wu, wd, operand_dtype=torch.bfloat16))
