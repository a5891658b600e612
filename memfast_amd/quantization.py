"""Read geometry, imported-parameter handling, packing, and the inverse of the quantizers.

Quantization itself runs only in the gfx950 kernels of libmemfast_hip.so:
``input_tiles`` and ``weight_tiles`` below (memfast/quantization.py:82-137) quantize
rectangular scale groups with IEEE division and round-half-even, bit for bit as the
reference's CPU routine does, and write the codes straight into array tiles.  There
is no host quantizer in this package.

What remains here is tensor bookkeeping around those kernels:
* the read geometry: which read every physical row belongs to and where each read
  starts (memfast/quantization.py:76-79);
* imported scales and zero points for ``Simulator.map_quantized``: broadcasting and
  validation (memfast/quantization.py:47-73) and packing of imported integer codes
  (memfast/quantization.py:94-112);
* dequantization, codes times their read's scale, which the hardware-aware training
  surrogate uses instead of quantizing its operands a second time.
"""

import math

import torch

from . import hip


# ---------------------------------------------------------------------------
# Read geometry
# ---------------------------------------------------------------------------
def row_reads(rows, config, device):
    """Index of the ADC read (array i, read j -> i*Gr + j) holding each of ``rows`` rows."""
    row = torch.arange(rows, device=device)
    array_rows = config.array_size[0]
    return row // array_rows * config.reads_per_array + row % array_rows // config.read_rows


def read_starts(partitions, config, device):
    """First physical row of each ADC read of ``partitions`` arrays (quantization.py:76-79)."""
    read = torch.arange(partitions * config.reads_per_array, device=device)
    per_array = config.reads_per_array
    return read // per_array * config.array_size[0] + read % per_array * config.read_rows


def check_read_scales(value, config, name):
    """Reject a [rows, cols] scale or zero-point table that changes inside one ADC read."""
    reads = row_reads(value.shape[0], config, value.device)
    starts = read_starts(math.ceil(value.shape[0] / config.array_size[0]), config, value.device)
    if not torch.equal(value, value[starts[reads]]):
        raise ValueError(f"{name} changes inside an ADC read; reduce rows_per_read")


# ---------------------------------------------------------------------------
# Imported parameters (Simulator.map_quantized)
# ---------------------------------------------------------------------------
def expanded_parameter(value, shape, device, dtype, name, *, positive=False):
    """Broadcast a scalar or tensor parameter to ``shape`` in ``dtype``; the reference's
    checks (memfast/quantization.py:47-64): real and finite as given, nonnegative when
    ``positive``, broadcastable, and still finite after the cast."""
    suffix = " and nonnegative" if positive else ""
    given = torch.as_tensor(value, device=device,
                            dtype=None if torch.is_tensor(value) else torch.float64)
    if given.is_complex() or not bool(torch.isfinite(given).all()):
        raise ValueError(f"{name} must be real and finite")
    if positive and bool((given < 0).any()):
        raise ValueError(f"{name} must be finite and nonnegative")
    try:
        cast = torch.broadcast_to(given.to(dtype), shape)
    except RuntimeError:
        raise ValueError(f"{name} must broadcast to {tuple(shape)}") from None
    if not bool(torch.isfinite(cast).all()) or (positive and bool((cast < 0).any())):
        raise ValueError(f"{name} must be finite{suffix}")
    return cast


def pack_weight(code, scale, config):
    """Tiles of imported integer codes: packed [m, p, R, C] (two's complement masked to
    weight_bits) and per-read scales [m*Gr, p, C], taken at each read's first row; padded
    rows and columns repeat the last logical row's and column's scale
    (memfast/quantization.py:94-112).  No scale is estimated."""
    k, o = code.shape
    rows, cols = config.array_size
    m, p = math.ceil(k / rows), math.ceil(o / cols)
    grid = code.new_zeros((m * rows, p * cols))
    grid[:k, :o] = code & ((1 << config.weight_bits) - 1)
    store = torch.int64 if config.wide_codes else torch.uint8
    packed = grid.view(m, rows, p, cols).transpose(1, 2).contiguous().to(store)
    table = scale.to(torch.float64 if config.wide else torch.float32)
    first_rows = read_starts(m, config, code.device).clamp_max(k - 1)
    columns = torch.arange(p * cols, device=code.device).clamp_max(o - 1)
    scales = table[first_rows][:, columns]
    return packed, scales.reshape(m * config.reads_per_array, p, cols).contiguous()


# ---------------------------------------------------------------------------
# The gfx950 quantizers and their inverse
# ---------------------------------------------------------------------------
def weight_tiles(weight, config):
    """PyTorch-layout [O,K] weights -> (packed [m,p,R,C], scales [m*Gr,p,C]) on the GPU."""
    packed, _, scales = hip.weight_tiles(weight, config, transposed=False)
    return packed, scales


def input_tiles(value, config, fixed_scale=None):
    """[N,K] inputs -> (codes [N,m,R], per-read scales [N,m*Gr]) on the GPU."""
    return hip.input_tiles(value, config, fixed_scale)


def _signed(codes, bits):
    """Two's complement ``bits``-bit codes (any integer storage) as int32 values."""
    value = codes.to(torch.int64) & ((1 << bits) - 1)
    return (value ^ (1 << (bits - 1))) - (1 << (bits - 1))


def dequantize_inputs(q, xscale, config, k):
    """Codes q [N, m, R] and per-read scales [N, m*Gr] -> FP32 values [N, k].

    Equals code * scale of the reference's grouped quantizer for every row (scale
    groups never cross a read, so a row's read scale is its group scale), formed in the
    scale's precision and rounded to FP32 as memfast/nn/training.py:62-72 does."""
    codes = _signed(q.reshape(q.shape[0], -1)[:, :k], config.activation_bits)
    scales = xscale[:, row_reads(k, config, q.device)]
    return (codes.to(scales.dtype) * scales).float()


def dequantize_program(packed, weight_scale, config, k, o):
    """A program's packed codes [m, p, R, C] and read scales [m*Gr, p, C] -> FP32 [k, o]
    physical weights (codes are signed unless ``config.weight_signed`` is False)."""
    m, p, rows, cols = packed.shape
    grid = packed.transpose(1, 2).reshape(m * rows, p * cols)[:k, :o]
    if config.weight_signed:
        codes = _signed(grid, config.weight_bits)
    else:
        codes = grid.to(torch.int64) & ((1 << config.weight_bits) - 1)
    table = weight_scale.reshape(m * config.reads_per_array, p * cols)[:, :o]
    scales = table[row_reads(k, config, packed.device)]
    return (codes.to(scales.dtype) * scales).float()


__all__ = [
    "row_reads", "read_starts", "check_read_scales", "expanded_parameter", "pack_weight",
    "weight_tiles", "input_tiles", "dequantize_inputs", "dequantize_program",
]
