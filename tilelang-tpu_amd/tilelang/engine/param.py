"""Kernel parameter metadata (reference tilelang/engine/param.py:13-109: dtype + static shape)."""
from dataclasses import dataclass
from typing import Any, List, Union

import torch

from ..utils.tensor import map_torch_type


@dataclass
class KernelParam:
    dtype: torch.dtype
    shape: List[Union[int, Any]]  # an int, or a symbolic extent (T.symbolic) bound per call

    @classmethod
    def from_buffer(cls, buffer) -> "KernelParam":
        from ..language import ir
        shape = []
        for s in buffer.shape:
            try:
                shape.append(int(ir.const_value(s)))
            except (TypeError, ValueError):
                shape.append(s)
        return cls(map_torch_type(buffer.dtype), shape)

    def is_dynamic(self) -> bool:
        return any(not isinstance(s, int) for s in self.shape)

    def is_scalar(self) -> bool:
        return len(self.shape) == 0

    def is_unsigned(self) -> bool:
        return str(self.dtype).replace("torch.", "").startswith("uint")

    def is_float8(self) -> bool:
        return "float8" in str(self.dtype)

    def is_boolean(self) -> bool:
        return self.dtype == torch.bool
