"""Framework bindings (reference python/tiga/interop/): ``tiga.interop.torch``."""

from . import torch

__all__ = ["torch"]
