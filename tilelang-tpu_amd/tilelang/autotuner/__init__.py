"""Autotuning is out of scope (tile shapes are fixed per kernel). The module exists because the
reference's MLA example does ``from tilelang.autotuner import *``
(examples/deepseek_mla/example_mla_decode_paged.py:3)."""
__all__ = []
