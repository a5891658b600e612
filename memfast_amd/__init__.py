"""memfast_amd: MI355X-native bit-sliced analog in-memory computing simulation.

Drop-in for MemFast's public API (memfast/__init__.py:3-20): ``import
memfast_amd as memfast``.  Products execute in hand-written gfx950 HIP kernels
(libmemfast_hip.so, bound by memfast_amd.hip); there is no CPU execution path.
"""

from .config import Config, Nonidealities
from .functional import matmul, mm
from .nn import AnalogConv2d, AnalogLinear, convert_model, reset_read_events
from .simulator import AnalogMatrix, Simulator

__version__ = "0.3.0"
__all__ = [
    "Config", "Nonidealities", "Simulator", "mm", "matmul", "AnalogMatrix", "AnalogLinear",
    "AnalogConv2d", "convert_model", "reset_read_events",
]
