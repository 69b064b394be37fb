"""JITKernel: the object ``tilelang.compile`` returns (reference tilelang/jit/kernel.py:21-387)."""
from typing import Any, Callable, Dict, List, Literal, Optional, Union

from ..engine.param import KernelParam
from ..profiler import Profiler
from ..utils.target import determine_target
from ..utils.tensor import TensorSupplyType
from .adapter.mi355x import MI355XKernelAdapter, recognize


SYMBOLIC_TRIAL = 4096  # trial value of each symbolic extent at compile time


class JITKernel:
    """Compiled kernel. Calling it runs the gfx950 kernel chosen for the program."""

    artifact = None

    def __init__(self, func=None, out_idx: Union[List[int], int, None] = None,
                 execution_backend: Literal["dlpack", "ctypes", "cython"] = "cython",
                 target: Union[str, Any] = "auto", target_host: Union[str, Any] = None,
                 verbose: bool = False, pass_configs: Optional[Dict[str, Any]] = None,
                 from_database: bool = False, mode: Literal["pcie", "cmodel"] = "pcie"):
        if execution_backend not in ("dlpack", "ctypes", "cython"):
            raise AssertionError(f"Invalid execution backend. {execution_backend}")
        if mode not in ("pcie", "cmodel"):
            raise AssertionError(f"Invalid execution mode. {mode}")
        self.execution_backend = execution_backend
        self.target = determine_target(target)
        self.target_host = target_host
        self.verbose = verbose
        self.pass_configs = pass_configs or {}
        self.mode = mode  # accepted for signature compatibility; there is one device path
        if from_database:
            return
        if func is None:
            raise ValueError("JITKernel needs a prim_func")
        self.prim_func = func
        sym = func.symbolic_vars() if hasattr(func, "symbolic_vars") else []
        # symbolic extents (T.symbolic): the program is recognised here at a trial binding, so
        # an unsupported program still fails at compile time; each call specialises it to the
        # argument shapes
        plan = recognize(func.specialize({n: SYMBOLIC_TRIAL for n in sym}) if sym else func)
        params = [KernelParam.from_buffer(b) for b in func.params]
        self.adapter = MI355XKernelAdapter(params, out_idx, plan, func)
        self.torch_function = self.adapter.func
        if verbose:
            print(f"[tilelang/mi355x] {func.name} -> {plan.describe()}")

    def __call__(self, *args: Any, **kwds: Any) -> Any:
        return self.torch_function(*args, **kwds)

    @property
    def func(self) -> Callable:
        """The adapter's callable. examples/deepseek_mla/benchmark_mla.py:446 calls
        ``kernel.func(...)``, which the reference's JITKernel lacks; it is provided here."""
        return self.adapter.func

    @property
    def plan(self):
        return self.adapter.plan

    def get_profiler(self, tensor_supply_type: TensorSupplyType = TensorSupplyType.Auto):
        return Profiler(self.params, self.out_idx,
                        tensor_supply_type).with_default_adapter(self.adapter)

    def get_kernel_source(self) -> str:
        return self.adapter.get_kernel_source()

    def get_host_source(self) -> str:
        return ""

    def run_once(self, func: Optional[Callable] = None):
        return self.get_profiler().run_once(func)

    @property
    def out_idx(self) -> List[int]:
        return self.adapter.result_idx

    @property
    def params(self) -> List[KernelParam]:
        return self.adapter.params

    @property
    def kernel_source(self) -> str:
        return self.adapter.get_kernel_source()

    @property
    def host_source(self) -> str:
        return ""
