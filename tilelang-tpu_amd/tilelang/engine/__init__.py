from .param import KernelParam  # noqa: F401
