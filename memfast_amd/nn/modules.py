"""``Linear`` and ``Conv2d`` with torch.nn's constructor signatures, an analog forward and
surrogate gradients (the reference's memfast/nn/modules.py).

Each layer is a hardware-aware layer (memfast_amd/nn/training.py) built around a fresh
``nn.Linear``/``nn.Conv2d`` made with the caller's arguments, so initialisation,
parameter shapes and dtypes are torch's.  On top of it:

* simulator options are keyword-only; a supplied simulator must agree with them;
* the programmed matrices are derived state: ``state_dict`` holds only ``weight`` and
  ``bias``, and loading reprograms the matrices from the loaded parameters;
* ``update_weight`` copies new weights into the existing Parameter and reprograms every
  convolution group, checking all groups before anything changes;
* moving the layer to another device moves its matrices to a simulator there;
* ``Conv2d`` accepts string paddings ("same"/"valid") and unbatched CHW inputs.
"""

import itertools
import math
from pathlib import Path

import torch
from torch import nn
from torch.nn import functional as F

from ..simulator import AnalogMatrix, Simulator
from .training import TrainableAnalogConv2d, TrainableAnalogLinear

_layer_ids = itertools.count()


def _layer_name():
    return f"layer.{next(_layer_ids)}"


def _simulator_for(simulator, config, device, mode, cache_dir):
    """The caller's simulator checked against the other options, or a new one."""
    if simulator is None:
        return Simulator(config, device="cuda" if device is None else device, mode=mode,
                         cache_dir=cache_dir)
    if not isinstance(simulator, Simulator):
        raise TypeError("simulator must be Simulator")
    if config is not None and config != simulator.config:
        raise ValueError("config differs from the supplied simulator")
    if device is not None:
        wanted = torch.device(device)
        if wanted.type == "cuda" and wanted.index is None:
            wanted = torch.device("cuda", torch.cuda.current_device())
        if wanted != simulator.device:
            raise ValueError("device differs from the supplied simulator")
    if mode != "default" and mode != simulator.mode:
        raise ValueError("mode differs from the supplied simulator")
    if cache_dir is not None and Path(cache_dir) != simulator.cache_dir:
        raise ValueError("cache_dir differs from the supplied simulator")
    return simulator


def _hide_programs(module, state, prefix, local_metadata):
    """State-dict hook: drop the programmed child's entries."""
    hidden = f"{prefix}{module._programs_attr}."
    for key in [key for key in state if key.startswith(hidden)]:
        del state[key]


class _ConstructorLayer:
    """What ``Linear`` and ``Conv2d`` add to the hardware-aware layers."""

    _programs_attr = None     # attribute of the programmed child module

    def _hide_programs_from_state(self):
        self.register_state_dict_post_hook(_hide_programs)

    @property
    def simulator(self):
        return next(self._programs())[0].simulator

    def state_dict(self, *args, **kwargs):
        if len(args) > 3:
            raise TypeError("state_dict accepts at most three positional arguments")
        kwargs.update(zip(("destination", "prefix", "keep_vars"), args))
        return super().state_dict(**kwargs)

    def _load_from_state_dict(self, state_dict, prefix, *args):
        super()._load_from_state_dict(state_dict, prefix, *args)
        self.update_weight()
        # The hidden child loads the state just programmed, so that strict loading finds
        # its keys and its own checks run.
        child = getattr(self, self._programs_attr)
        for key, value in child.state_dict(prefix=f"{prefix}{self._programs_attr}.").items():
            state_dict.setdefault(key, value)

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse=recurse)
        programs = [module for module in self.modules() if isinstance(module, AnalogMatrix)]
        if programs and programs[0].simulator.device != self.weight.device:
            relocated = programs[0].simulator._relocated(self.weight.device)
            for program in programs:
                program.simulator = relocated
                program._prepared.clear()
        return self

    def _checked_replacement(self, weight):
        if not isinstance(weight, torch.Tensor) or weight.shape != self.weight.shape:
            raise ValueError("weight must have the layer's original PyTorch shape")
        if not weight.is_floating_point() or not bool(torch.isfinite(weight).all()):
            raise ValueError("weight must be real floating and finite")
        cast = weight.to(self.weight)
        if not bool(torch.isfinite(cast).all()):
            raise ValueError("weight exceeds the layer parameter dtype")
        if not self.simulator.config.weight_signed and bool((cast < 0).any()):
            raise ValueError("unsigned weights must be nonnegative")
        return cast

    @torch.no_grad()
    def update_weight(self, weight=None):
        """Copy optional PyTorch-layout weights into the Parameter and reprogram; every
        group is quantized and checked before the Parameter or any program changes."""
        replacement = None if weight is None else self._checked_replacement(weight)
        source = self.weight if replacement is None else replacement
        prepared = [(matrix, matrix._prepare(block, bias))
                    for matrix, block, bias in self._programs(source)]
        if replacement is not None:
            self.weight.copy_(replacement)
        for matrix, program in prepared:
            matrix._commit(program)
            matrix._prepared.clear()
        return self

    def reset_parameters(self):
        """torch.nn's initialisation (nonnegative weights for unsigned configurations),
        then reprogramming."""
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if not self.simulator.config.weight_signed:
            with torch.no_grad():
                self.weight.abs_()
        if self.bias is not None:
            fan_in, _ = nn.init._calculate_fan_in_and_fan_out(self.weight)
            limit = 1 / math.sqrt(fan_in) if fan_in else 0
            nn.init.uniform_(self.bias, -limit, limit)
        self.update_weight()


def _nonnegative_if_unsigned(source, config):
    if not config.weight_signed:
        with torch.no_grad():
            source.weight.abs_()
    return source


class Linear(_ConstructorLayer, TrainableAnalogLinear):
    """Linear(in_features, out_features, bias=True, device=None, dtype=None)."""

    _programs_attr = "matrix"

    def __init__(self, in_features, out_features, bias=True, device=None, dtype=None, *,
                 simulator=None, config=None, mode="default", cache_dir=None,
                 gradient_mode="quantized"):
        engine = _simulator_for(simulator, config, device, mode, cache_dir)
        source = nn.Linear(in_features, out_features, bias, device=engine.device, dtype=dtype)
        super().__init__(_nonnegative_if_unsigned(source, engine.config), engine,
                         name=_layer_name(), gradient_mode=gradient_mode)
        self._hide_programs_from_state()

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}")


class Conv2d(_ConstructorLayer, TrainableAnalogConv2d):
    """Conv2d with torch.nn's argument order and keyword-only simulator options."""

    _programs_attr = "analog"

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True, padding_mode="zeros", device=None, dtype=None, *,
                 simulator=None, config=None, mode="default", cache_dir=None,
                 gradient_mode="quantized"):
        engine = _simulator_for(simulator, config, device, mode, cache_dir)
        source = nn.Conv2d(in_channels, out_channels, kernel_size, stride, padding, dilation,
                           groups, bias, padding_mode, device=engine.device, dtype=dtype)
        # A string padding becomes an explicit pad of the input (torch's own amounts for
        # "same", which may be uneven) ahead of an unpadded convolution.
        input_padding = None
        if isinstance(padding, str):
            input_padding = (tuple(source._reversed_padding_repeated_twice),
                            "constant" if padding_mode == "zeros" else padding_mode)
            source.padding, source.padding_mode = (0, 0), "zeros"
        super().__init__(_nonnegative_if_unsigned(source, engine.config), engine,
                         name=_layer_name(), gradient_mode=gradient_mode)
        self._hide_programs_from_state()
        self._input_padding = input_padding
        self._requested_padding = padding

    def forward(self, input):
        batched = input.ndim != 3
        x = input if batched else input.unsqueeze(0)
        if self._input_padding is not None and any(self._input_padding[0]):
            x = F.pad(x, self._input_padding[0], mode=self._input_padding[1])
        output = super().forward(x)
        return output if batched else output.squeeze(0)

    def extra_repr(self):
        return (f"{self.in_channels}, {self.out_channels}, kernel_size={self.kernel_size}, "
                f"stride={self.stride}, padding={self._requested_padding!r}, "
                f"groups={self.groups}, bias={self.bias is not None}")


__all__ = ["Linear", "Conv2d"]
