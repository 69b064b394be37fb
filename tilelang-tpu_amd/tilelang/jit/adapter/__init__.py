from .base import BaseKernelAdapter  # noqa: F401
from .mi355x import MI355XKernelAdapter  # noqa: F401
