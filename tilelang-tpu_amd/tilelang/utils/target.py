"""Target strings (reference tilelang/utils/target.py:10-18, 47-92).

The reference accepts {"auto", "cuda", "hip", "webgpu", "c", "llvm", "tpu"}. Here every program
runs on gfx950, so "mi355x" is the canonical target; "auto", "hip", "rocm" and "tpu" are
accepted as aliases so that the reference's scripts (which pass target="tpu" or nothing) run
unmodified. Targets of other hardware are rejected.
"""
from typing import Union

MI355X = "mi355x"
AVAILABLE_TARGETS = {"auto", "mi355x", "hip", "rocm", "tpu", "gfx950"}
# Spelling kept from the reference (utils/target.py:10).
AVALIABLE_TARGETS = AVAILABLE_TARGETS


def determine_target(target: Union[str, object] = "auto", return_object: bool = False) -> str:
    t = getattr(target, "kind", None)
    t = getattr(t, "name", None) or str(target)
    t = t.split()[0].lower()
    if t not in AVAILABLE_TARGETS:
        raise ValueError(f"Target {target!r} is not supported: this build runs gfx950 (MI355X) "
                         f"only; use one of {sorted(AVAILABLE_TARGETS)}")
    return MI355X
