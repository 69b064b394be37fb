"""gfx950 execution backend: recogniser + ctypes dispatch into libtlmi355x.so."""
from .adapter import MI355XKernelAdapter  # noqa: F401
from .recognize import Plan, UnsupportedProgram, recognize  # noqa: F401
