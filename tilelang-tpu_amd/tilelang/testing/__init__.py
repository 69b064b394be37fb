"""Test helpers (reference tilelang/testing/__init__.py:20-25 for the seeding convention)."""
import random

import numpy as np
import torch

from ..utils.tensor import torch_assert_close  # noqa: F401


def set_random_seed(seed: int = 42) -> None:
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def requires_mi355x(fn):
    """Skip unless a gfx950 device is visible (the reference gates GPU tests the same way)."""
    import pytest
    ok = torch.cuda.is_available()
    if ok:
        name = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
        ok = name.startswith("gfx950")
    return pytest.mark.skipif(not ok, reason="needs an MI355X (gfx950)")(fn)
