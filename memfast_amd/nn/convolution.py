"""Convolution lowered to one programmed matrix per convolution group.

Restates memfast/nn/convolution.py: the input is unfolded into patches
(F.unfold) and each group's [N*L, Cin/g*kh*kw] patch matrix is read through
its own AnalogMatrix; stride, dilation, numeric padding, padding modes and
groups are preserved.
"""

import math

import torch
from torch import nn
from torch.nn import functional as F

_COPIED = ("in_channels", "out_channels", "kernel_size", "stride", "padding", "dilation",
           "groups", "padding_mode")


class AnalogConv2d(nn.Module):
    """Conv2d whose groups are independently programmed analog matrices."""

    def __init__(self, source, simulator, *, name="conv"):
        super().__init__()
        if not isinstance(source, nn.Conv2d):
            raise TypeError("source must be torch.nn.Conv2d")
        if isinstance(source.padding, str):
            raise ValueError("use numeric Conv2d padding before conversion")
        for attr in _COPIED:
            setattr(self, attr, getattr(source, attr))
        self.matrices = nn.ModuleList()
        per_group = source.out_channels // source.groups
        for group in range(source.groups):
            block = slice(group * per_group, (group + 1) * per_group)
            bias = None if source.bias is None else source.bias[block]
            self.matrices.append(
                simulator.map(source.weight[block].flatten(1), bias=bias, name=f"{name}.group{group}")
            )

    @torch.no_grad()
    def forward(self, x):
        if x.ndim != 4 or x.shape[1] != self.in_channels:
            raise ValueError("expected NCHW input with matching channels")
        height_in, width_in = x.shape[-2:]
        padding = self.padding
        if self.padding_mode != "zeros":
            ph, pw = padding
            x = F.pad(x, (pw, pw, ph, ph), mode=self.padding_mode)
            padding = (0, 0)
        patches = F.unfold(x, self.kernel_size, self.dilation, padding, self.stride)
        size = self.in_channels // self.groups * math.prod(self.kernel_size)
        outputs = [
            matrix(patches[:, g * size:(g + 1) * size].transpose(1, 2))
            for g, matrix in enumerate(self.matrices)
        ]
        merged = torch.cat(outputs, dim=-1).transpose(1, 2)
        spatial = [
            (extent + 2 * pad - dil * (kernel - 1) - 1) // step + 1
            for extent, pad, dil, kernel, step in zip(
                (height_in, width_in), self.padding, self.dilation, self.kernel_size, self.stride
            )
        ]
        return merged.reshape(x.shape[0], self.out_channels, *spatial)
