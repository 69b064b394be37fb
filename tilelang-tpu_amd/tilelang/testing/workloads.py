"""Seeded synthetic inputs for the benchmark configs (BASELINE.json ``configs``).

All tensors are generated on the host from ``torch.Generator().manual_seed(seed)`` and copied
to the device by the caller, so CPU and GPU see identical bits. ``scale`` shrinks the
configuration for quick parity runs (scale=1 is the full config).
"""
import math
from dataclasses import dataclass, field
from typing import Dict

import torch


@dataclass
class Workload:
    name: str
    tensors: Dict[str, torch.Tensor]
    attrs: Dict = field(default_factory=dict)

    def to(self, device):
        return Workload(self.name, {k: v.to(device) for k, v in self.tensors.items()},
                        dict(self.attrs))


def _g(seed):
    return torch.Generator().manual_seed(seed)


def rmsnorm(rows=4096, cols=4096, dtype=torch.float16, seed=0, eps=1e-6):
    g = _g(seed)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1.0 + 0.1 * torch.randn(cols, generator=g)).to(dtype)
    return Workload("rmsnorm", dict(x=x, w=w), dict(eps=eps, rows=rows, cols=cols))


def gemm(M=4096, N=4096, K=4096, dtype=torch.float16, seed=0):
    g = _g(seed)
    a = (torch.rand(M, K, generator=g) * 2 - 1).to(dtype)
    b = (torch.rand(K, N, generator=g) * 2 - 1).to(dtype)
    return Workload("gemm", dict(a=a, b=b), dict(M=M, N=N, K=K))


def rope(tokens=8192, heads=32, dim=128, dtype=torch.bfloat16, seed=0, base=10000.0):
    g = _g(seed)
    q = torch.randn(tokens, heads, dim, generator=g).to(dtype)
    k = torch.randn(tokens, heads, dim, generator=g).to(dtype)
    # fp32 angle tables, interleaved-duplicated (pairs 2i, 2i+1 share theta_i)
    i = torch.arange(dim // 2, dtype=torch.float32)
    inv = base ** (-2.0 * i / dim)
    theta = torch.arange(tokens, dtype=torch.float32)[:, None] * inv[None, :]
    cos = torch.repeat_interleave(torch.cos(theta), 2, dim=1).to(dtype).contiguous()
    sin = torch.repeat_interleave(torch.sin(theta), 2, dim=1).to(dtype).contiguous()
    return Workload("rope", dict(q=q, k=k, cos=cos, sin=sin), dict(tokens=tokens, heads=heads,
                                                                 dim=dim))


def swiglu(rows=8192, cols=14336, dtype=torch.bfloat16, seed=0):
    g = _g(seed)
    gate = torch.randn(rows, cols, generator=g).to(dtype)
    up = torch.randn(rows, cols, generator=g).to(dtype)
    return Workload("swiglu", dict(gate=gate, up=up), dict(rows=rows, cols=cols))


def flashattn(B=8, S=4096, H=32, D=128, causal=True, dtype=torch.bfloat16, seed=0):
    g = _g(seed)
    q = torch.randn(B, S, H, D, generator=g).to(dtype)
    k = torch.randn(B, S, H, D, generator=g).to(dtype)
    v = torch.randn(B, S, H, D, generator=g).to(dtype)
    return Workload("flashattn", dict(q=q, k=k, v=v), dict(B=B, S=S, H=H, D=D, causal=causal,
                                                           sm_scale=1.0 / math.sqrt(D)))


def mla(B=64, Hq=128, dv=512, dpe=64, page=64, max_pages=128, min_len=1024, max_len=8192,
        seed=0, q_dtype=torch.bfloat16):
    """DeepSeek-V3-style FP8 MLA decode inputs. KV pool has B*max_pages pages; the block table
    is a random permutation of all pages (every page distinct)."""
    g = _g(seed)
    lens = torch.randint(min_len, max_len + 1, (B,), generator=g, dtype=torch.int64)
    lens = torch.minimum(lens, torch.tensor(max_pages * page)).to(torch.int32)
    n_pages = B * max_pages
    table = torch.randperm(n_pages, generator=g).view(B, max_pages).to(torch.int32)
    latent = torch.randn(n_pages * page, dv + dpe, generator=g)
    scale = float(latent.abs().max()) / 448.0
    kv = (latent / scale).to(torch.float8_e4m3fn)
    del latent
    q = torch.randn(B, Hq, dv + dpe, generator=g).to(q_dtype)
    return Workload("mla", dict(q=q, kv=kv, block_table=table, seqlens=lens,
                                kv_scale=torch.tensor([scale], dtype=torch.float32)),
                    dict(B=B, Hq=Hq, dv=dv, dpe=dpe, page=page, max_pages=max_pages,
                         sm_scale=1.0 / math.sqrt(192.0)))
