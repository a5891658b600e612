"""Quantization and packing with independent rectangular scale groups.

Same public functions as the reference's memfast/quantization.py.  The hot
path (``weight_tiles``/``input_tiles``: quantize, slice-pack, gather per-read
scales) runs in the gfx950 kernels of libmemfast_hip.so with IEEE FP32
division and round-half-even, bit-identical to the reference CPU path.

``grouped_quantize`` remains a device-agnostic torch routine: the product
uses it only for the FP32 surrogate gradient of hardware-aware training
(memfast/nn/training.py:72-93), never for the analog forward.
"""

import math

import torch
from torch.nn import functional as F

from . import hip


def grouped_quantize(value, bits, granularity, bw_e=None, *, signed=True):
    """INT/BFP codes and expanded scales of rectangular groups (quantization.py:9-44)."""
    dtype = torch.float64 if bits > 8 or bw_e is not None else torch.float32
    value = value.to(dtype)
    if not torch.isfinite(value).all():
        raise ValueError(f"quantized values must be finite in {dtype}")
    if not signed and ((value < 0).any() or bw_e is not None):
        raise ValueError(
            "unsigned floating weights must be nonnegative INT values; "
            "use map_quantized with zero_points for affine weights"
        )
    rows, cols = value.shape
    gr = rows if granularity[0] is None else min(granularity[0], rows)
    gc = cols if granularity[1] is None else min(granularity[1], cols)
    nr, nc = math.ceil(rows / gr), math.ceil(cols / gc)
    blocks = F.pad(value, (0, nc * gc - cols, 0, nr * gr - rows)).reshape(nr, gr, nc, gc)
    peak = blocks.abs().amax((1, 3), keepdim=True)
    upper = (1 << (bits - int(signed))) - 1
    if bw_e is None:
        scale = torch.where(peak > 0, peak, torch.ones_like(peak)) / upper
        tiny = torch.finfo(dtype).smallest_normal * torch.finfo(dtype).eps
        scale = scale.clamp_min(tiny)
        lower = -upper if signed else 0
    else:
        limit = (1 << (bw_e - 1)) - 1
        exponent = peak.clamp_min(torch.finfo(dtype).tiny).log2().floor().clamp(1 - limit, limit)
        scale = torch.pow(2.0, exponent + 2 - bits)
        lower = -(1 << (bits - 1))
    code = (blocks / scale).round().clamp_(lower, upper)
    code = code.reshape(nr * gr, nc * gc)[:rows, :cols].to(torch.int64)
    full = scale.expand(nr, gr, nc, gc).reshape(nr * gr, nc * gc)[:rows, :cols]
    return code, full


def expanded_parameter(value, shape, device, dtype, name, *, positive=False):
    """Broadcast a scalar/tensor parameter to ``shape`` with finiteness checks."""
    if torch.is_tensor(value):
        original = torch.as_tensor(value, device=device)
    else:
        original = torch.as_tensor(value, device=device, dtype=torch.float64)
    if original.is_complex() or not torch.isfinite(original).all():
        raise ValueError(f"{name} must be real and finite")
    if positive and (original < 0).any():
        raise ValueError(f"{name} must be finite and nonnegative")
    converted = original.to(dtype)
    try:
        converted = torch.broadcast_to(converted, shape)
    except RuntimeError:
        raise ValueError(f"{name} must broadcast to {tuple(shape)}") from None
    if not torch.isfinite(converted).all() or (positive and (converted < 0).any()):
        raise ValueError(f"{name} must be finite" + (" and nonnegative" if positive else ""))
    return converted


def check_read_scales(value, config, name):
    """Reject scales or zero points that change inside one ADC read."""
    rows = config.array_size[0]
    index = torch.arange(value.shape[0], device=value.device)
    start = (index // rows) * rows + ((index % rows) // config.read_rows) * config.read_rows
    if not torch.equal(value, value[start]):
        raise ValueError(f"{name} changes inside an ADC read; reduce rows_per_read")


def read_starts(partitions, config, device):
    """First physical row of each ADC read (quantization.py:76-79)."""
    base = torch.arange(partitions, device=device)[:, None] * config.array_size[0]
    offsets = torch.arange(config.reads_per_array, device=device)[None] * config.read_rows
    return (base + offsets).flatten()


def pack_weight(code, scale, config):
    """Pack logical [K,O] integer codes (no scale estimation); quantization.py:94-112.

    Integer masking and reshaping only, so it is exact on any device.
    """
    k, o = code.shape
    r, c = config.array_size
    m, p = math.ceil(k / r), math.ceil(o / c)
    scale = scale.to(torch.float64 if config.wide else torch.float32)
    padded = F.pad(code, (0, p * c - o, 0, m * r - k))
    store = torch.int64 if config.wide_codes else torch.uint8
    packed = (padded & ((1 << config.weight_bits) - 1)).to(store)
    packed = packed.reshape(m, r, p, c).permute(0, 2, 1, 3).contiguous()
    grown = F.pad(scale[None, None], (0, p * c - o, 0, m * r - k), mode="replicate")[0, 0]
    scales = grown[read_starts(m, config, code.device)]
    return packed, scales.reshape(m * config.reads_per_array, p, c).contiguous()


def weight_tiles(weight, config):
    """PyTorch-layout [O,K] weights -> (packed [m,p,R,C], scales [m*Gr,p,C]) on the GPU."""
    packed, _, scales = hip.weight_tiles(weight, config, transposed=False)
    return packed, scales


def input_tiles(value, config, fixed_scale=None):
    """[N,K] inputs -> (codes [N,m,R], per-read scales [N,m*Gr]) on the GPU."""
    return hip.input_tiles(value, config, fixed_scale)


__all__ = [
    "grouped_quantize", "expanded_parameter", "check_read_scales", "read_starts",
    "pack_weight", "weight_tiles", "input_tiles",
]
