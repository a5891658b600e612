"""Does this host's torch CPU ``sum`` add the reads in the order the read kernels reproduce?

The reference restores and sums a chunk's reads with ``value.sum(1)`` on a
contiguous [N, G, width, C] tensor (memfast/simulator.py:582-585), FP32 or FP64
for wide configurations.  The read kernels of libmemfast_hip.so reproduce the
order in which torch's CPU kernel performs that reduction, so that their outputs
equal the reference's bit for bit:

* the columns inside whole spans of a chunk (32 FP32 columns, 4 when the chunk is
  narrower than 8; 16 FP64 columns) sum the reads as a cascade: blocks of 2^L reads
  (L = max(4, ceil(log2 G) / 4)) are summed sequentially, each full block is added
  into the next level, recursively, and the levels are combined lowest first;
* the remaining columns sum four interleaved cascades (reads g = k mod 4, over
  G / 4 reads each), add the leftover reads to the first and fold the four.

That layout matches torch 2.x on hosts whose ``torch.backends.cpu.get_cpu_capability()``
reports "AVX512" (an Intel Xeon and an AMD EPYC), and with torch's kernels forced to
"AVX2" and "DEFAULT" (``ATEN_CPU_CAPABILITY``) on them: the order does not depend on the
vector ISA.  A host whose torch reduces in another order computes reference outputs
that differ from the kernels' in the last bits.

``sum_order_matches()`` probes torch on this host once per process, FP32 and FP64, on
columns of both classes; the ``Simulator`` constructor warns when it does not match.
"""

import warnings
from functools import lru_cache

import torch

VERIFIED_CAPABILITIES = ("AVX512", "AVX2", "DEFAULT")


def _level_power(reads):
    return max(4, max(1, (reads - 1).bit_length()) // 4)


def cascade_sum(values):
    """Sum [G, W] ``values`` over G in the kernels' cascade order (adds in their dtype)."""
    reads = values.shape[0]
    power = _level_power(reads)
    mask = (1 << power) - 1
    levels = [torch.zeros(values.shape[1:], dtype=values.dtype) for _ in range(4)]
    for count in range(1, reads + 1):
        levels[0] = levels[0] + values[count - 1]
        if count & mask == 0:
            for level in range(1, 4):
                levels[level] = levels[level] + levels[level - 1]
                levels[level - 1] = torch.zeros_like(levels[level - 1])
                if count & (mask << (level * power)):
                    break
    total = levels[0]
    for level in range(1, 4):
        total = total + levels[level]
    return total


def interleaved_sum(values):
    """Sum [G, W] ``values`` over G as four interleaved cascades (reads g = k mod 4), the
    leftover reads added to the first, then the four folded in order."""
    reads = values.shape[0]
    full = reads // 4 * 4
    zero = torch.zeros(values.shape[1:], dtype=values.dtype)
    if not full:
        total = zero
        for g in range(reads):
            total = total + values[g]
        return total
    streams = [cascade_sum(values[k:full:4]) for k in range(4)]
    total = streams[0]
    for g in range(full, reads):
        total = total + values[g]
    for k in (1, 2, 3):
        total = total + streams[k]
    return total


def kernel_order_sum(values):
    """Sum one chunk's [G, W] ``values`` over G with the kernels' column classes."""
    width = values.shape[1]
    span = 16 if values.dtype == torch.float64 else (32 if width >= 8 else 4)
    cut = width // span * span
    parts = []
    if cut:
        parts.append(cascade_sum(values[:, :cut]))
    if cut < width:
        parts.append(interleaved_sum(values[:, cut:]))
    return torch.cat(parts)


def probe_values(reads=300, columns=64, dtype=torch.float32):
    """Reads with magnitudes spread over 2^-20..2^20, so that summation orders differ."""
    generator = torch.Generator().manual_seed(1234)
    base = torch.randn(1, reads, columns, generator=generator)
    spread = torch.randint(-20, 21, (1, reads, columns), generator=generator).float()
    return (base * torch.exp2(spread)).to(dtype)


@lru_cache(maxsize=1)
def sum_order_matches():
    """True when torch's CPU sum over reads equals ``kernel_order_sum`` bit for bit here,
    in FP32 (72 columns: 64 cascade, 8 interleaved) and FP64 (40: 32 and 8)."""
    for columns, dtype, view in ((72, torch.float32, torch.int32),
                                 (40, torch.float64, torch.int64)):
        values = probe_values(columns=columns, dtype=dtype)
        expected = kernel_order_sum(values[0])
        if not torch.equal(values.sum(1)[0].view(view), expected.view(view)):
            return False
    return True


@lru_cache(maxsize=1)
def warn_if_different():
    """Warn once per process when this host's torch CPU sum order differs from the kernels'."""
    if sum_order_matches():
        return True
    warnings.warn(
        "torch's CPU sum on this host (capability "
        f"{torch.backends.cpu.get_cpu_capability()}) adds reads in another order than the "
        "read kernels reproduce (verified on "
        f"{', '.join(VERIFIED_CAPABILITIES)}); the reference's CPU outputs on this host may "
        "differ from memfast_amd's in the last bits",
        RuntimeWarning, stacklevel=3)
    return False
