"""Tensor helpers: dtype map, input supply and the tolerance check.

Semantics follow the reference's tilelang/utils/tensor.py: ``map_torch_type`` (:24-32),
``TensorSupplyType`` and its generators (:14-122), ``torch_assert_close`` with an allowed
mismatch ratio (:212-300).
"""
from enum import Enum

import torch


class TensorSupplyType(Enum):
    Integer = 1
    Uniform = 2
    Normal = 3
    Randn = 4
    Zero = 5
    One = 6
    Auto = 7


_TORCH = {
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "float32": torch.float32,
    "float64": torch.float64,
    "int32": torch.int32,
    "int64": torch.int64,
    "int8": torch.int8,
    "uint8": torch.uint8,
    "uint32": torch.uint32,
    "bool": torch.bool,
    "float8_e4m3": torch.float8_e4m3fn,
    "float8_e5m2": torch.float8_e5m2,
}


def map_torch_type(intype) -> torch.dtype:
    if isinstance(intype, torch.dtype):
        return intype
    from ..language.ir import canon_dtype
    return _TORCH[canon_dtype(intype)]


def get_tensor_supply(supply_type: TensorSupplyType):
    """Return ``param -> tensor`` on the current HIP device for the given supply type."""

    def get_tensor(param) -> torch.Tensor:
        if param.is_scalar():  # as the reference's supply (tilelang/utils/tensor.py)
            raise ValueError(f"TensorType must have a shape, but got {type(param)}: scalar "
                             "parameters have no random supply; pass the inputs explicitly")
        dtype = param.dtype
        shape = [int(s) for s in param.shape]
        device = torch.device("cuda", torch.cuda.current_device())
        st = supply_type
        is_float = dtype in (torch.float16, torch.bfloat16, torch.float32)
        if param.is_float8():
            return torch.randint(-128, 128, shape, device=device, dtype=torch.int8).to(dtype) \
                if st in (TensorSupplyType.Auto, TensorSupplyType.Integer) else \
                torch.randn(*shape, device=device).to(dtype)
        if st == TensorSupplyType.Auto:
            if param.is_unsigned():
                return torch.randint(0, 3, shape, device=device, dtype=dtype)
            if param.is_boolean():
                return torch.randint(0, 2, shape, device=device, dtype=dtype)
            if is_float:
                return torch.empty(*shape, device=device, dtype=dtype).normal_(-1.0, 1.0)
            return torch.randint(-2, 3, shape, device=device, dtype=dtype)
        if dtype == torch.int8 and st in (TensorSupplyType.Uniform, TensorSupplyType.Normal):
            return torch.ones(*shape, device=device, dtype=dtype)
        if st == TensorSupplyType.Integer:
            if param.is_unsigned():
                return torch.randint(0, 3, shape, device=device, dtype=dtype)
            return torch.randint(-2, 3, shape, device=device, dtype=dtype)
        if st == TensorSupplyType.Uniform:
            return torch.empty(*shape, device=device, dtype=dtype).uniform_(-1.0, 1.0)
        if st == TensorSupplyType.Normal:
            return torch.empty(*shape, device=device, dtype=dtype).normal_(-1.0, 1.0)
        if st == TensorSupplyType.Randn:
            return torch.randn(*shape, device=device).to(dtype)
        if st == TensorSupplyType.Zero:
            return torch.zeros(*shape, device=device, dtype=dtype)
        if st == TensorSupplyType.One:
            return torch.ones(*shape, device=device, dtype=dtype)
        raise NotImplementedError(st)

    return get_tensor


def torch_assert_close(tensor_a, tensor_b, rtol=1e-2, atol=1e-3, max_mismatched_ratio=0.001,
                       verbose=False, equal_nan=True, check_device=True, check_dtype=True,
                       **kwargs):
    """Assert ``|a-b| <= atol + rtol*|b|`` for all but ``max_mismatched_ratio`` of elements."""
    if tensor_a.shape != tensor_b.shape:
        raise AssertionError(f"shape mismatch: {tuple(tensor_a.shape)} != {tuple(tensor_b.shape)}")
    if check_dtype and tensor_a.dtype != tensor_b.dtype:
        raise AssertionError(f"dtype mismatch: {tensor_a.dtype} != {tensor_b.dtype}")
    if check_device and tensor_a.device != tensor_b.device:
        raise AssertionError(f"device mismatch: {tensor_a.device} != {tensor_b.device}")
    a = tensor_a.detach().cpu().to(torch.float64)
    b = tensor_b.detach().cpu().to(torch.float64)
    bad = ~torch.isclose(a, b, rtol=rtol, atol=atol, equal_nan=equal_nan)
    nbad = int(bad.sum())
    allowed = int(a.numel() * max_mismatched_ratio)
    if verbose:
        print(f"mismatched {nbad} / {a.numel()} (allowed {allowed})")
    if nbad > allowed:
        flat = int(bad.reshape(-1).to(torch.int8).argmax())
        diff = (a - b).abs()
        raise AssertionError(
            f"Too many mismatched elements: {nbad} > {allowed} "
            f"({max_mismatched_ratio * 100:.2f}% allowed). First mismatch at flat index {flat}: "
            f"lhs={a.reshape(-1)[flat].item():.6f}, rhs={b.reshape(-1)[flat].item():.6f}. "
            f"Greatest absolute difference: {diff.max().item()}.")
    return True
