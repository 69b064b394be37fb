"""Profiler (reference tilelang/profiler/__init__.py:22-229): input supply, tolerance check
against a reference program, consistency reruns, and timing."""
from functools import partial
from typing import Any, Callable, List, Optional

import torch

from ..utils.tensor import TensorSupplyType, get_tensor_supply, torch_assert_close
from .bench import do_bench  # noqa: F401


def _as_list(outs) -> list:
    if outs is None:
        return []
    return [outs] if isinstance(outs, torch.Tensor) else list(outs)


class Profiler:

    def __init__(self, params, result_idx, supply_type=TensorSupplyType.Auto, adapter=None):
        from ..jit.adapter.base import legalize_result_idx
        self.params = params
        self.result_idx = legalize_result_idx(result_idx, len(params))
        self.supply_type = supply_type
        self.supply = get_tensor_supply(supply_type)
        self.adapter = adapter

    def with_default_adapter(self, adapter) -> "Profiler":
        self.adapter = adapter
        return self

    def _get_inputs(self, with_output=False):
        return [self.supply(p) for i, p in enumerate(self.params)
                if with_output or i not in self.result_idx]

    def _get_params(self, with_output=False):
        return [p for i, p in enumerate(self.params) if with_output or i not in self.result_idx]

    def assert_allclose(self, reference_program: Callable,
                        input_tensors: Optional[List[torch.Tensor]] = None, atol: float = 1e-2,
                        rtol: float = 1e-2, max_mismatched_ratio=0.01):
        """Run the kernel and ``reference_program`` on the same inputs (generated from the
        parameters unless given) and require every output pair to agree within atol + rtol |ref|
        on all but ``max_mismatched_ratio`` of the elements."""
        args = self._get_inputs() if input_tensors is None else input_tensors
        expected = _as_list(reference_program(*args))
        torch.cuda.synchronize()
        got = _as_list(self.func(*args))
        torch.cuda.synchronize()
        if len(got) != len(expected):
            raise AssertionError(f"the kernel returned {len(got)} outputs and the reference "
                                 f"program {len(expected)}")
        for out, exp in zip(got, expected):
            torch_assert_close(out, exp, rtol=rtol, atol=atol,
                               max_mismatched_ratio=max_mismatched_ratio)

    def assert_consistent(self, repeat=10):
        """Rerun on the same inputs and require bitwise-identical outputs (race check)."""
        ins = self._get_inputs()
        ref = self.func(*ins)
        ref = [ref] if isinstance(ref, torch.Tensor) else ref
        ref = [r.clone() for r in ref]
        for _ in range(repeat):
            outs = self.func(*ins)
            outs = [outs] if isinstance(outs, torch.Tensor) else outs
            for a, b in zip(outs, ref):
                assert torch.equal(a, b), "result is not consistent"

    def run_once(self, func: Optional[Callable] = None):
        ins = self._get_inputs()
        return (func or self.__call__)(*ins)

    def do_bench(self, func: Optional[Callable] = None, warmup: int = 25, rep: int = 100,
                 n_warmup: int = 1, n_repeat: int = 1, input_tensors=None) -> float:
        if func is None:
            assert self.adapter is not None, "benchmarking function should be provided"
            func = self.adapter
        ins = self._get_inputs() if input_tensors is None else input_tensors
        return do_bench(partial(func, *ins), warmup=warmup, rep=rep, _n_warmup=n_warmup,
                        _n_repeat=n_repeat)

    @property
    def func(self):
        assert self.adapter is not None, "adapter should be provided"
        return self.adapter

    def __call__(self, *args: Any, **kwds: Any) -> Any:
        return self.func(*args, **kwds)
