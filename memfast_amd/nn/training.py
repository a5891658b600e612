"""Hardware-aware training: analog forward values, surrogate gradients.

Behaviour of memfast/nn/training.py.  A trainable layer keeps ordinary master
Parameters.  Every forward writes the current parameters into the layer's programmed
matrices in place (identities of parameters and buffers never change, so optimizers
and distributed wrappers see stable objects), reads the matrices on the GPU, and, when
gradients are wanted, ties the analog values to a surrogate whose gradient backward
uses:

* ``gradient_mode="quantized"`` (default): the surrogate multiplies dequantized
  operands, and the quantizers pass gradients through unchanged.  dx therefore uses the
  dequantized grouped weights and dw the dequantized grouped inputs.  The weights'
  values are the program just written (its codes times their read scales).  The inputs'
  values come from the GPU quantizer's codes and read scales under dynamic grouped
  scales, whatever fixed scale the forward read used;
* ``gradient_mode="digital"``: the unquantized layer's derivatives.

Neither mode differentiates device effects (noise, faults, the ADC).  The surrogate
computes in FP32 with autocast off, and gradients reach leaf Parameters in their own
dtype.  Convolutions form their surrogate on unfolded patches, one programmed matrix
per group, so input gradients fold back over overlapping patches.
"""

import torch
from torch import nn
from torch.nn import functional as F

from .. import hip
from ..quantization import dequantize_inputs, dequantize_program
from .convolution import AnalogConv2d

GRADIENT_MODES = ("quantized", "digital")


def _validate_gradient_mode(mode):
    if not isinstance(mode, str) or mode not in GRADIENT_MODES:
        raise ValueError("gradient_mode must be quantized or digital")
    return mode


class _SurrogateGradient(torch.autograd.Function):
    """Forward passes the analog value through; backward hands the incoming gradient to
    the surrogate (in the surrogate's dtype) and none to the analog value."""

    @staticmethod
    def forward(ctx, analog, surrogate):
        ctx.surrogate_dtype = surrogate.dtype
        return analog

    @staticmethod
    def backward(ctx, grad_output):
        return None, grad_output.to(ctx.surrogate_dtype)


def _through(value, replacement):
    """``replacement``'s values with the identity derivative with respect to ``value``."""
    return value + (replacement - value).detach()


@torch.no_grad()
def _dequantized_inputs(flat, config):
    """FP32 grouped-quantized values of ``flat`` [N, K] (dynamic scales), from the GPU
    quantizer's codes and read scales."""
    if flat.numel() == 0:
        return flat.float()
    q, xscale = hip.input_tiles(flat.detach(), config)
    return dequantize_inputs(q, xscale, config, flat.shape[1])


@torch.no_grad()
def _dequantized_weights(matrix):
    """FP32 physical [K, O] weights of ``matrix``'s current program."""
    return dequantize_program(matrix.packed, matrix.weight_scale, matrix.config,
                              matrix.in_features, matrix.out_features)


def _linear_surrogate(x, weight, bias, matrix):
    """Quantized-operand surrogate of ``x @ weight.T + bias`` read through ``matrix``
    (programmed from ``weight``); leading dimensions of ``x`` are flattened first."""
    flat = x.reshape(-1, matrix.in_features).float()
    inputs = _through(flat, _dequantized_inputs(flat, matrix.config))
    weights = _through(weight.float().T, _dequantized_weights(matrix))
    value = inputs @ weights
    if bias is not None:
        value = value + bias.float()
    return value.reshape(*x.shape[:-1], matrix.out_features)


def _master(value, device):
    """A trainable copy of a source layer's Parameter on ``device`` (None stays None)."""
    if value is None:
        return None
    return nn.Parameter(value.detach().to(device).clone(), requires_grad=value.requires_grad)


class _HardwareAware(nn.Module):
    """Shared forward of the trainable layers: program, read, attach the surrogate.

    Subclasses provide ``_programs`` (each programmed matrix with its block of the
    master parameters), ``_read`` (the analog forward of detached inputs) and the two
    surrogates."""

    def _program(self):
        """Write the master parameters into the programmed matrices."""
        for matrix, weight, bias in self._programs():
            matrix._reprogram(weight, bias)

    def forward(self, x):
        with torch.autocast(device_type=x.device.type, enabled=False):
            self._program()
            analog = self._read(x.detach())
            if not torch.is_grad_enabled():
                return analog
            surrogate = (self._quantized_surrogate(x) if self.gradient_mode == "quantized"
                         else self._digital_surrogate(x))
        return _SurrogateGradient.apply(analog, surrogate)


class TrainableAnalogLinear(_HardwareAware):
    """``nn.Linear`` with an analog forward and surrogate gradients."""

    def __init__(self, source, simulator, *, name="linear", gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.Linear):
            raise TypeError("source must be torch.nn.Linear")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self.in_features, self.out_features = source.in_features, source.out_features
        self.weight = _master(source.weight, simulator.device)
        self.register_parameter("bias", _master(source.bias, simulator.device))
        self.matrix = simulator.map(self.weight, bias=self.bias, name=name)
        self.train(source.training)

    def _programs(self, weight=None):
        yield self.matrix, self.weight if weight is None else weight, self.bias

    def _read(self, x):
        return self.matrix(x)

    def _quantized_surrogate(self, x):
        return _linear_surrogate(x, self.weight, self.bias, self.matrix)

    def _digital_surrogate(self, x):
        return F.linear(x.float(), self.weight.float(),
                        None if self.bias is None else self.bias.float())


_CONV_ATTRIBUTES = ("in_channels", "out_channels", "kernel_size", "stride", "padding",
                    "dilation", "groups", "padding_mode")


class TrainableAnalogConv2d(_HardwareAware):
    """Grouped ``nn.Conv2d`` with an analog forward and surrogate gradients."""

    def __init__(self, source, simulator, *, name="conv", gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.Conv2d):
            raise TypeError("source must be torch.nn.Conv2d")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self.weight = _master(source.weight, simulator.device)
        self.register_parameter("bias", _master(source.bias, simulator.device))
        self.analog = AnalogConv2d(source, simulator, name=name)
        for attribute in _CONV_ATTRIBUTES:
            setattr(self, attribute, getattr(source, attribute))
        self.train(source.training)

    def _programs(self, weight=None):
        """(matrix, [O/g, Cin/g*kh*kw] block of ``weight`` (the master weight by default),
        bias block or None) of every convolution group."""
        weight = self.weight if weight is None else weight
        width = self.out_channels // self.groups
        for group, matrix in enumerate(self.analog.matrices):
            rows = slice(group * width, (group + 1) * width)
            yield matrix, weight[rows].flatten(1), None if self.bias is None else self.bias[rows]

    def _read(self, x):
        return self.analog(x)

    def _padded(self, x):
        """FP32 input and the padding left for unfold/conv2d (non-zero padding modes pad
        explicitly, as the analog forward does)."""
        x = x.float()
        if self.padding_mode == "zeros":
            return x, self.padding
        ph, pw = self.padding
        return F.pad(x, (pw, pw, ph, ph), mode=self.padding_mode), (0, 0)

    def _quantized_surrogate(self, x):
        source, padding = self._padded(x)
        patches = F.unfold(source, self.kernel_size, self.dilation, padding, self.stride)
        size = self.weight[0].numel()
        pieces = [
            _linear_surrogate(patches[:, g * size:(g + 1) * size].transpose(1, 2), weight, bias,
                              matrix)
            for g, (matrix, weight, bias) in enumerate(self._programs())
        ]
        merged = torch.cat(pieces, dim=-1).transpose(1, 2)
        spatial = [(extent + 2 * pad - dil * (k - 1) - 1) // step + 1
                   for extent, pad, dil, k, step in zip(x.shape[-2:], self.padding, self.dilation,
                                                        self.kernel_size, self.stride)]
        return merged.reshape(x.shape[0], self.out_channels, *spatial)

    def _digital_surrogate(self, x):
        source, padding = self._padded(x)
        return F.conv2d(source, self.weight.float(),
                        None if self.bias is None else self.bias.float(), self.stride, padding,
                        self.dilation, self.groups)


__all__ = ["TrainableAnalogLinear", "TrainableAnalogConv2d", "GRADIENT_MODES"]
