from .target import determine_target, AVALIABLE_TARGETS, AVAILABLE_TARGETS  # noqa: F401
from .tensor import TensorSupplyType, map_torch_type, torch_assert_close  # noqa: F401
