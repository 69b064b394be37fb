"""Adapter base: output-index legalisation (reference tilelang/jit/adapter/base.py:20-44)."""
from typing import Any, Callable, List, Optional, Union


def legalize_result_idx(result_idx: Optional[Union[int, List[int]]], n_params: int) -> List[int]:
    """``None`` -> []; an int or a list of ints in [-n, n-1] -> non-negative indices."""
    if result_idx is None:
        return []
    if isinstance(result_idx, int):
        result_idx = [result_idx]
    if not isinstance(result_idx, (list, tuple)):
        raise ValueError("result_idx should be a list of integers")
    out = []
    for idx in result_idx:
        if not isinstance(idx, int) or idx >= n_params or idx < -n_params:
            raise ValueError(
                f"result_idx should be an integer between {-n_params} and {n_params - 1}, "
                f"got {idx}")
        out.append(idx + n_params if idx < 0 else idx)
    return out


class BaseKernelAdapter:
    func: Optional[Callable] = None

    def __init__(self, mod, params, result_idx) -> None:
        self.mod = mod
        self.params = params
        self.result_idx = legalize_result_idx(result_idx, len(params))
        self.func = self._convert_torch_func()

    def _legalize_result_idx(self, result_idx):
        return legalize_result_idx(result_idx, len(self.params))

    def _convert_torch_func(self) -> Callable:
        raise NotImplementedError

    def __call__(self, *args: Any, **kwds: Any) -> Any:
        return self.func(*args, **kwds)
