"""Does this host's torch CPU ``sum`` add the reads in the order the read kernels reproduce?

The reference restores and sums a chunk's reads with ``value.sum(1)`` on a
contiguous [N, G, width, C] FP32 tensor (memfast/simulator.py:582-585).  The
read kernels of libmemfast_hip.so reproduce the order in which torch's CPU
kernel performs that reduction, so that their outputs equal the reference's
bit for bit: blocks of 2^L reads (L = max(4, ceil(log2 G) / 4)) are summed
sequentially, each full block is added into the next level, recursively, and
the levels are combined lowest first.  That layout was verified on hosts where
``torch.backends.cpu.get_cpu_capability()`` reports "AVX512" (an Intel Xeon
and an AMD EPYC).  A host whose torch reduces in another order computes
reference outputs that differ from the kernels' in the last bits.

``sum_order_matches()`` probes torch on this host once per process; the
``Simulator`` constructor warns when it does not match.
"""

import warnings
from functools import lru_cache

import torch

VERIFIED_CAPABILITIES = ("AVX512",)


def _level_power(reads):
    return max(4, max(1, (reads - 1).bit_length()) // 4)


def cascade_sum(values):
    """Sum [G, W] FP32 ``values`` over G in the kernels' order (FP32 adds, read by read)."""
    reads = values.shape[0]
    power = _level_power(reads)
    mask = (1 << power) - 1
    levels = [torch.zeros(values.shape[1:], dtype=torch.float32) for _ in range(4)]
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


def probe_values(reads=300, columns=64):
    """Reads with magnitudes spread over 2^-20..2^20, so that summation orders differ."""
    generator = torch.Generator().manual_seed(1234)
    base = torch.randn(1, reads, columns, generator=generator)
    spread = torch.randint(-20, 21, (1, reads, columns), generator=generator).float()
    return (base * torch.exp2(spread)).float()


@lru_cache(maxsize=1)
def sum_order_matches():
    """True when torch's CPU sum over reads equals ``cascade_sum`` bit for bit here."""
    values = probe_values()
    expected = cascade_sum(values[0])
    return torch.equal(values.sum(1)[0].view(torch.int32), expected.view(torch.int32))


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
