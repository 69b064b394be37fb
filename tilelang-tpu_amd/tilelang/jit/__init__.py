"""``tilelang.compile`` / ``tilelang.jit`` (reference tilelang/jit/__init__.py:24-133).

The reference routes ``compile`` through a kernel cache whose lookup is disabled
(tilelang/cache/kernel_cache.py:137-185), so every call builds a fresh kernel; here a compile is
a trace recognition plus a ctypes binding, so it is equally uncached and cheap.
"""
from typing import Any, Dict, List, Literal, Optional, Union

from .kernel import JITKernel


def compile(func=None, out_idx: Union[List[int], int, None] = None,
            execution_backend: Literal["dlpack", "ctypes", "cython"] = "cython",
            target: Union[str, Any] = "auto", target_host: Union[str, Any] = None,
            verbose: bool = False, pass_configs: Optional[Dict[str, Any]] = None,
            mode: Literal["pcie", "cmodel"] = "pcie") -> JITKernel:
    return JITKernel(func, out_idx=out_idx, execution_backend=execution_backend, target=target,
                     target_host=target_host, verbose=verbose, pass_configs=pass_configs,
                     mode=mode)


def jit(func=None, *, out_idx=None, execution_backend="cython", target="auto", target_host=None,
        verbose=False, pass_configs=None, mode="pcie"):

    def deco(f):
        return compile(f, out_idx=out_idx, execution_backend=execution_backend, target=target,
                       target_host=target_host, verbose=verbose, pass_configs=pass_configs,
                       mode=mode)

    return deco(func) if func is not None else deco
