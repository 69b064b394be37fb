"""Layout surface. The reference's swizzled layouts (tilelang/layout/, src/layout/) drive GPU
codegen; the gfx950 kernels here use fixed LDS layouts, so these calls are accepted and ignored
(``make_swizzled_layout`` is called by examples/deepseek_mla/example_mla_decode_paged.py:48-51)."""
from ..language import Fragment, Layout  # noqa: F401


def make_swizzled_layout(buffer, *args, **kwargs):
    return Layout(getattr(buffer, "shape", None))
