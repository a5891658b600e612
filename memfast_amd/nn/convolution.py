"""Convolution lowered to one programmed matrix per convolution group.

Restates memfast/nn/convolution.py: each group's [N*L, Cin/g*kh*kw] patch
matrix (F.unfold's) is read through its own AnalogMatrix; stride, dilation,
numeric padding, padding modes and groups are preserved.  In default mode a
narrow configuration never builds the patch matrix: the input quantizer
gathers each patch element straight from the NCHW image (implicit im2col),
which yields the same codes and scales.
"""

import math

import torch
from torch import nn
from torch.nn import functional as F

from .. import hip

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
        spatial = [
            (extent + 2 * pad - dil * (kernel - 1) - 1) // step + 1
            for extent, pad, dil, kernel, step in zip(
                (height_in, width_in), self.padding, self.dilation, self.kernel_size, self.stride
            )
        ]
        outputs = self._implicit(x, padding, spatial)
        if outputs is None:
            patches = F.unfold(x, self.kernel_size, self.dilation, padding, self.stride)
            size = self.in_channels // self.groups * math.prod(self.kernel_size)
            outputs = [
                matrix(patches[:, g * size:(g + 1) * size].transpose(1, 2))
                for g, matrix in enumerate(self.matrices)
            ]
        merged = (outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=-1)).transpose(1, 2)
        return merged.reshape(x.shape[0], self.out_channels, *spatial)

    def _implicit(self, x, padding, spatial):
        """Per-group outputs [N, L, O/groups] read from implicit-im2col input tiles, or
        None where the patch matrix path applies (tuned mode, wide configurations, and
        inputs that AnalogMatrix.forward rejects, so it raises its own error)."""
        first = self.matrices[0]
        config = first.config
        scale_dtype = torch.float32
        if (first.simulator.mode != "default" or config.wide or x.numel() == 0
                or not x.is_floating_point() or min(spatial) < 1
                or x.device != first.packed.device or x.device != first.simulator.device
                or any(m.weight_scale.dtype != scale_dtype for m in self.matrices)):
            return None
        per_group = self.in_channels // self.groups
        size = per_group * math.prod(self.kernel_size)
        rows = spatial[0] * spatial[1]
        meta = torch.empty((x.shape[0], rows, size), dtype=x.dtype, device="meta")
        value = x.to(torch.float32).contiguous()
        outputs = []
        for g, matrix in enumerate(self.matrices):
            status = hip.status_word(x.device)
            geometry = (g * per_group, per_group, self.kernel_size, self.stride, padding,
                        self.dilation, spatial)
            q, xscale = hip.conv_input_tiles(value, config, geometry, matrix.input_scale,
                                             status=status)
            outputs.append(matrix._run(meta, q, xscale, status=status))
        return outputs
