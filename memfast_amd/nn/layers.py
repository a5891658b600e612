"""Compatibility imports of the Linear and Conv2d adapters (memfast/nn/layers.py)."""

from .convolution import AnalogConv2d
from .linear import AnalogLinear

__all__ = ["AnalogLinear", "AnalogConv2d"]
