"""Hardware-aware training: analog forward values, FP32 surrogate gradients.

Restates memfast/nn/training.py.  Master weights and biases are ordinary
Parameters; every forward reprograms the persistent analog buffers from them
(so parameter and buffer identities stay stable for optimizers), runs the
analog kernels, and attaches a surrogate whose gradient is used in backward:

* ``gradient_mode="quantized"`` (default): dx uses dequantized grouped
  weights, dw uses dequantized grouped inputs, quantizers pass gradients
  through unchanged;
* ``gradient_mode="digital"``: derivatives of the unquantized digital layer.

Neither mode differentiates device effects.  Surrogate arithmetic is FP32.
"""

import torch
from torch import nn
from torch.nn import functional as F

from ..quantization import grouped_quantize
from .convolution import AnalogConv2d


class _SurrogateGradient(torch.autograd.Function):
    """Forward returns the analog value; backward routes the gradient to the surrogate."""

    @staticmethod
    def forward(ctx, analog, surrogate):
        ctx.surrogate_dtype = surrogate.dtype
        return analog

    @staticmethod
    def backward(ctx, grad_output):
        return None, grad_output.to(ctx.surrogate_dtype)


@torch.no_grad()
def _program(matrix, weight, bias):
    """Reprogram ``matrix`` in place, keeping its name, read counter and selections."""
    fresh = matrix.simulator.map(weight, bias=bias, name=matrix.name)
    matrix.packed.copy_(fresh.packed)
    matrix.weight_scale.copy_(fresh.weight_scale)
    if matrix.bias is not None:
        matrix.bias.copy_(fresh.bias)
    matrix._kernel_codes = fresh._kernel_codes if fresh._kernel_codes is None else (
        matrix._codes_key(), fresh._kernel_codes[1]
    )


def _parameter(value, device):
    if value is None:
        return None
    return nn.Parameter(value.detach().to(device).clone(), requires_grad=value.requires_grad)


def _validate_gradient_mode(mode):
    if not isinstance(mode, str) or mode not in ("quantized", "digital"):
        raise ValueError("gradient_mode must be quantized or digital")
    return mode


def _quantized_operand(value, bits, granularity, config, reference=None, *, signed=True):
    """Straight-through dequantized operand in FP32."""
    operand = value.float()
    if value.numel() == 0:
        return operand
    with torch.no_grad():
        source = value if reference is None else reference
        code, scale = grouped_quantize(source.detach(), bits, granularity, config.bw_e,
                                       signed=signed)
        dequantized = (code * scale).float()
    return operand + (dequantized - operand).detach()


def _quantized_linear(x, weight, bias, config, input_reference=None):
    """FP32 surrogate of the analog linear map: quantized inputs @ quantized weights."""
    flat = x.reshape(-1, weight.shape[1])
    reference = None if input_reference is None else input_reference.reshape(-1, weight.shape[1])
    inputs = _quantized_operand(flat, config.activation_bits, config.input_quant_gran, config,
                                reference=reference)
    weights = _quantized_operand(weight.T, config.weight_bits, config.weight_quant_gran, config,
                                 signed=config.weight_signed)
    output = inputs @ weights
    if bias is not None:
        output = output + bias.to(output.dtype)
    return output.reshape(*x.shape[:-1], weight.shape[0])


class TrainableAnalogLinear(nn.Module):
    """Linear layer with an analog forward and a selectable STE backward."""

    def __init__(self, source, simulator, *, name="linear", gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.Linear):
            raise TypeError("source must be torch.nn.Linear")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self.in_features, self.out_features = source.in_features, source.out_features
        self.weight = _parameter(source.weight, simulator.device)
        self.register_parameter("bias", _parameter(source.bias, simulator.device))
        self.matrix = simulator.map(self.weight, bias=self.bias, name=name)
        self.train(source.training)

    def forward(self, x):
        with torch.autocast(device_type=x.device.type, enabled=False):
            _program(self.matrix, self.weight, self.bias)
            analog = self.matrix(x.detach())
            if not torch.is_grad_enabled():
                return analog
            if self.gradient_mode == "quantized":
                surrogate = _quantized_linear(x, self.weight, self.bias, self.matrix.config)
            else:
                bias = None if self.bias is None else self.bias.float()
                surrogate = F.linear(x.float(), self.weight.float(), bias)
        return _SurrogateGradient.apply(analog, surrogate)


class TrainableAnalogConv2d(nn.Module):
    """Grouped Conv2d with an analog forward and a selectable STE backward."""

    def __init__(self, source, simulator, *, name="conv", gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.Conv2d):
            raise TypeError("source must be torch.nn.Conv2d")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self.weight = _parameter(source.weight, simulator.device)
        self.register_parameter("bias", _parameter(source.bias, simulator.device))
        self.analog = AnalogConv2d(source, simulator, name=name)
        for attr in ("in_channels", "out_channels", "kernel_size", "stride", "padding",
                     "dilation", "groups", "padding_mode"):
            setattr(self, attr, getattr(source, attr))
        self.train(source.training)

    def forward(self, x):
        with torch.autocast(device_type=x.device.type, enabled=False):
            return self._forward(x)

    def _forward(self, x):
        per_group = self.out_channels // self.groups
        for group, matrix in enumerate(self.analog.matrices):
            block = slice(group * per_group, (group + 1) * per_group)
            bias = None if self.bias is None else self.bias[block]
            _program(matrix, self.weight[block].flatten(1), bias)
        analog = self.analog(x.detach())
        if not torch.is_grad_enabled():
            return analog
        original = x.detach()
        x = x.float()
        padding = self.padding
        if self.padding_mode != "zeros":
            ph, pw = padding
            x = F.pad(x, (pw, pw, ph, ph), mode=self.padding_mode)
            original = F.pad(original, (pw, pw, ph, ph), mode=self.padding_mode)
            padding = (0, 0)
        if self.gradient_mode == "quantized":
            patches = F.unfold(x, self.kernel_size, self.dilation, padding, self.stride)
            reference = (
                patches.detach() if original.dtype == torch.float32
                else F.unfold(original, self.kernel_size, self.dilation, padding, self.stride)
            )
            size = self.weight[0].numel()
            pieces = []
            for group, matrix in enumerate(self.analog.matrices):
                block = slice(group * per_group, (group + 1) * per_group)
                bias = None if self.bias is None else self.bias[block]
                cols = slice(group * size, (group + 1) * size)
                pieces.append(_quantized_linear(
                    patches[:, cols].transpose(1, 2), self.weight[block].flatten(1), bias,
                    matrix.config, input_reference=reference[:, cols].transpose(1, 2),
                ))
            surrogate = torch.cat(pieces, dim=-1).transpose(1, 2).reshape(analog.shape)
        else:
            bias = None if self.bias is None else self.bias.float()
            surrogate = F.conv2d(x, self.weight.float(), bias, self.stride, padding,
                                 self.dilation, self.groups)
        return _SurrogateGradient.apply(analog, surrogate)
