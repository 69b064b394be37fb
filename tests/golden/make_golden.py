"""Write tests/golden/golden.npz: small seeded cases for every kernel family.

The reference commits no input/output vectors for this path, so these fixtures are produced by
this repository's oracle (oracle/ref.py, itself pinned by tests/test_oracle.py). They freeze the
oracle's outputs (tests/test_golden.py re-derives them bit for bit on the CPU) and give the GPU
kernels fixed vectors to match. 16-bit floats are stored as raw uint16 bits, fp8 as raw uint8.

Usage: python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tilelang-tpu_amd"))

from oracle import ref  # noqa: E402
from tilelang.testing import workloads  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.contiguous().view(torch.uint8).numpy()
    return t.contiguous().numpy()


def cases():
    out = {}
    w = workloads.rmsnorm(8, 512, seed=101)
    out["rmsnorm_x"], out["rmsnorm_w"] = bits(w.tensors["x"]), bits(w.tensors["w"])
    out["rmsnorm_y"] = bits(ref.rmsnorm_ref(w.tensors["x"], w.tensors["w"], 1e-6))
    w = workloads.gemm(32, 48, 64, seed=102)
    out["gemm_a"], out["gemm_b"] = bits(w.tensors["a"]), bits(w.tensors["b"])
    out["gemm_c"] = bits(ref.matmul_ref(w.tensors["a"], w.tensors["b"]))
    w = workloads.rope(4, 2, 64, seed=103)
    for n in ("q", "k", "cos", "sin"):
        out[f"rope_{n}"] = bits(w.tensors[n])
    out["rope_q_out"] = bits(ref.rope_ref(w.tensors["q"], w.tensors["cos"], w.tensors["sin"]))
    out["rope_k_out"] = bits(ref.rope_ref(w.tensors["k"], w.tensors["cos"], w.tensors["sin"]))
    w = workloads.swiglu(16, 40, seed=104)
    out["swiglu_gate"], out["swiglu_up"] = bits(w.tensors["gate"]), bits(w.tensors["up"])
    out["swiglu_out"] = bits(ref.swiglu_ref(w.tensors["gate"], w.tensors["up"]))
    w = workloads.flashattn(1, 40, 2, 64, causal=True, seed=105)
    for n in ("q", "k", "v"):
        out[f"fa_{n}"] = bits(w.tensors[n])
    out["fa_o"] = bits(ref.flashattn_ref(w.tensors["q"], w.tensors["k"], w.tensors["v"], True))
    w = workloads.mla(B=2, Hq=64, page=16, max_pages=4, min_len=1, max_len=64, seed=106)
    T = w.tensors
    out["mla_q"], out["mla_kv"] = bits(T["q"]), bits(T["kv"])
    out["mla_block_table"], out["mla_seqlens"] = T["block_table"].numpy(), T["seqlens"].numpy()
    out["mla_kv_scale"] = T["kv_scale"].numpy()
    out["mla_o"] = bits(ref.mla_decode_ref(T["q"][..., :512], T["q"][..., 512:],
                                           T["kv"][:, :512], T["kv"][:, 512:], T["block_table"],
                                           T["seqlens"], 16, 1 / math.sqrt(192),
                                           float(T["kv_scale"])))
    return out


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **cases())
    print("wrote", os.path.join(HERE, "golden.npz"))
