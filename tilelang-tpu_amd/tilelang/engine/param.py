"""Kernel parameter metadata (reference tilelang/engine/param.py:13-109: dtype + static shape)."""
from dataclasses import dataclass
from typing import List

import torch

from ..utils.tensor import map_torch_type


@dataclass
class KernelParam:
    dtype: torch.dtype
    shape: List[int]

    @classmethod
    def from_buffer(cls, buffer) -> "KernelParam":
        return cls(map_torch_type(buffer.dtype), [int(s) for s in buffer.shape])

    def is_scalar(self) -> bool:
        return len(self.shape) == 0

    def is_unsigned(self) -> bool:
        return str(self.dtype).replace("torch.", "").startswith("uint")

    def is_float8(self) -> bool:
        return "float8" in str(self.dtype)

    def is_boolean(self) -> bool:
        return self.dtype == torch.bool
