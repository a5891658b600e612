"""Convolution on programmed matrices, one per convolution group (memfast/nn/convolution.py).

Group g's weights [O/groups, Cin/groups*kh*kw] are one programmed matrix, read with the
group's patch matrix: F.unfold's [N*L, Cin/groups*kh*kw] rows for that group's input
channels.  Stride, dilation, numeric padding, the padding modes and groups are kept.

The patch matrix itself is never built where it can be avoided: the input quantizer
gathers each patch element straight from the NCHW image (implicit im2col,
``hip.conv_input_tiles``), which yields the same codes and scales as quantizing the
unfolded matrix.  This covers default and tuned mode and narrow and wide
configurations.  Only inputs that the read itself would reject (and empty outputs) take
the unfold route, so that the matrix raises its own error.
"""

import math

import torch
from torch import nn
from torch.nn import functional as F

from .. import hip

_COPIED = ("in_channels", "out_channels", "kernel_size", "stride", "padding", "dilation",
           "groups", "padding_mode")


def _output_size(extent, padding, dilation, kernel, stride):
    return [(size + 2 * pad - dil * (k - 1) - 1) // step + 1
            for size, pad, dil, k, step in zip(extent, padding, dilation, kernel, stride)]


class AnalogConv2d(nn.Module):
    """Conv2d whose groups are independently programmed analog matrices."""

    def __init__(self, source, simulator, *, name="conv"):
        super().__init__()
        if not isinstance(source, nn.Conv2d):
            raise TypeError("source must be torch.nn.Conv2d")
        if isinstance(source.padding, str):
            raise ValueError("use numeric Conv2d padding before conversion")
        for attribute in _COPIED:
            setattr(self, attribute, getattr(source, attribute))
        width = source.out_channels // source.groups
        self.matrices = nn.ModuleList()
        for group in range(source.groups):
            rows = slice(group * width, (group + 1) * width)
            self.matrices.append(simulator.map(
                source.weight[rows].flatten(1), name=f"{name}.group{group}",
                bias=None if source.bias is None else source.bias[rows]))

    @property
    def _patch_width(self):
        return self.in_channels // self.groups * math.prod(self.kernel_size)

    @torch.no_grad()
    def forward(self, x):
        if x.ndim != 4 or x.shape[1] != self.in_channels:
            raise ValueError("expected NCHW input with matching channels")
        spatial = _output_size(x.shape[-2:], self.padding, self.dilation, self.kernel_size,
                               self.stride)
        padding = self.padding
        if self.padding_mode != "zeros":
            # Non-zero padding modes pad explicitly; the patches then need none.
            ph, pw = padding
            x = F.pad(x, (pw, pw, ph, ph), mode=self.padding_mode)
            padding = (0, 0)
        if self._gathers(x, spatial):
            groups = self._gathered(x, padding, spatial)
        else:
            groups = self._unfolded(x, padding)
        merged = groups[0] if len(groups) == 1 else torch.cat(groups, dim=-1)
        return merged.transpose(1, 2).reshape(x.shape[0], self.out_channels, *spatial)

    def _unfolded(self, x, padding):
        """Per-group outputs [N, L, O/groups] read from F.unfold's patch matrix."""
        patches = F.unfold(x, self.kernel_size, self.dilation, padding, self.stride)
        width = self._patch_width
        return [matrix(patches[:, g * width:(g + 1) * width].transpose(1, 2))
                for g, matrix in enumerate(self.matrices)]

    def _gathers(self, x, spatial):
        """Whether the input tiles can be gathered from the image: inputs every
        matrix accepts (AnalogMatrix.forward's checks) and a non-empty output."""
        first = self.matrices[0]
        scale_dtype = torch.float64 if first.config.wide else torch.float32
        return (x.numel() > 0 and x.is_floating_point() and min(spatial) >= 1
                and x.device == first.packed.device == first.simulator.device
                and all(m.weight_scale.dtype == scale_dtype for m in self.matrices))

    def _gathered(self, x, padding, spatial):
        """Per-group outputs [N, L, O/groups] read from input tiles gathered from ``x``.

        Default mode leaves the finiteness check to the read's status word; tuned mode
        checks it before the schedule search, as the read of an unfolded matrix does."""
        per_group = self.in_channels // self.groups
        # Stands in for the patch rows where only their shape and dtype matter.
        patch_shape = torch.empty((x.shape[0], spatial[0] * spatial[1], self._patch_width),
                                  dtype=x.dtype, device="meta")
        outputs = []
        for g, matrix in enumerate(self.matrices):
            geometry = (g * per_group, per_group, self.kernel_size, self.stride, padding,
                        self.dilation, spatial)
            deferred = matrix.simulator.mode == "default"
            status = hip.status_word(x.device) if deferred else None
            q, xscale = hip.conv_input_tiles(x, matrix.config, geometry, matrix.input_scale,
                                             status=status)
            outputs.append(matrix._run(patch_shape, q, xscale, status=status))
        return outputs
