"""tilelang for MI355X (gfx950).

A drop-in for the kernel path of TileLang-TPU: programs written with ``tilelang.language``
(``T.prim_func``, ``T.Kernel``, ``T.ppl_*`` ...) compile with
``tilelang.compile(func, out_idx=-1, target="mi355x")`` into a callable over torch tensors
that runs hand-written gfx950 HIP kernels (libtlmi355x.so). Targets "auto" and "tpu" are
accepted as aliases so the reference's scripts run unmodified.
"""
import logging

__version__ = "0.1.0+mi355x"

logger = logging.getLogger("tilelang")


def set_log_level(level):
    logger.setLevel(level)


from . import language  # noqa: E402,F401
from . import layout  # noqa: E402,F401
from .engine.param import KernelParam  # noqa: E402,F401
from .jit import JITKernel, compile, jit  # noqa: E402,F401
from .profiler import Profiler  # noqa: E402,F401
from .utils.target import determine_target  # noqa: E402,F401
from .utils.tensor import TensorSupplyType  # noqa: E402,F401
from .jit.adapter.mi355x import UnsupportedProgram  # noqa: E402,F401


def lower(*args, **kwargs):
    """TIR lowering is replaced by recognition (see ``tilelang.compile``)."""
    raise NotImplementedError("tilelang.lower: there is no TIR lowering on the mi355x target; "
                              "use tilelang.compile")
