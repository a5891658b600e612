"""The read-summation order the HIP epilogue implements equals torch's CPU ``sum``.

memfast/simulator.py:585 sums (T*xs)*ws over reads with ``value.sum(1)`` on a
[N, G, width*C] tensor (width = 2 tiles per chunk).  The kernels
(memfast_amd/csrc/mf_device.h Cascade/Interleaved, and the column classes of
memfast_amd/csrc/general.hip) reproduce that order incrementally, read by read.
This test restates that incremental algorithm in Python and checks it bit for
bit against torch on this machine's CPU.
"""

import numpy as np
import pytest
import torch


def ceil_log2(x):
    return 1 if x <= 2 else (x - 1).bit_length()


def level_power(size):
    return max(4, ceil_log2(size) // 4)


class Cascade:
    def __init__(self, shape):
        self.acc = [np.zeros(shape, np.float32) for _ in range(4)]
        self.count = 0

    def push(self, x, lp):
        self.acc[0] = (self.acc[0] + x).astype(np.float32)
        self.count += 1
        step_mask = (1 << lp) - 1
        if self.count & step_mask == 0:
            for j in range(1, 4):
                self.acc[j] = (self.acc[j] + self.acc[j - 1]).astype(np.float32)
                self.acc[j - 1] = np.zeros_like(self.acc[j - 1])
                if self.count & (step_mask << (j * lp)):
                    break

    def finish(self):
        r = self.acc[0]
        for j in range(1, 4):
            r = (r + self.acc[j]).astype(np.float32)
        return r


def interleaved_sum(values):
    total = values.shape[0]
    full = (total // 4) * 4
    lp = level_power(total // 4)
    streams = [Cascade(values.shape[1:]) for _ in range(4)]
    first = np.zeros(values.shape[1:], np.float32)
    for g in range(total):
        if g < full:
            streams[g & 3].push(values[g], lp)
            if g + 1 == full:
                first = streams[0].finish()
        else:
            first = (first + values[g]).astype(np.float32)
    if full:
        for k in (1, 2, 3):
            first = (first + streams[k].finish()).astype(np.float32)
    return first


def cascade_sum(values):
    c = Cascade(values.shape[1:])
    lp = level_power(values.shape[0])
    for g in range(values.shape[0]):
        c.push(values[g], lp)
    return c.finish()


def interleaved_column(pos, wc):
    span = 32 if wc >= 8 else 4
    return pos >= (wc // span) * span


def kernel_sum(values):
    """values [G, wc]: per-column class dispatch as in the kernels."""
    wc = values.shape[1]
    out = np.empty(wc, np.float32)
    for col in range(wc):
        column = values[:, col:col + 1]
        out[col] = (interleaved_sum(column) if interleaved_column(col, wc)
                    else cascade_sum(column))[0]
    return out


@pytest.mark.parametrize("wc", [4, 5, 8, 12, 16, 24, 32, 36, 40, 48, 64, 68, 96, 100, 128, 144,
                                256])
@pytest.mark.parametrize("groups", [1, 3, 4, 5, 15, 16, 17, 33, 64, 100, 128, 255, 256, 300])
def test_kernel_order_matches_torch(wc, groups):
    gen = torch.Generator().manual_seed(groups * 1000 + wc)
    x = torch.randn(2, groups, wc, generator=gen) * torch.exp(3 * torch.randn(2, groups, wc,
                                                                               generator=gen))
    x = x.float()
    expected = x.sum(1).numpy()
    for n in range(2):
        got = kernel_sum(x[n].numpy())
        np.testing.assert_array_equal(got.view(np.int32), expected[n].view(np.int32))


def test_large_read_counts():
    """Level 2 of the cascade (>= 256 reads) and odd tails."""
    for groups in (511, 512, 1024, 1030):
        gen = torch.Generator().manual_seed(groups)
        x = (torch.randn(1, groups, 64, generator=gen) * 1e3).float()
        np.testing.assert_array_equal(kernel_sum(x[0].numpy()).view(np.int32),
                                      x.sum(1)[0].numpy().view(np.int32))


def test_host_capability_and_order_probe():
    """Record this host's torch CPU capability and check the product's probe: torch's sum
    here follows the cascade the kernels reproduce (memfast_amd/host_order.py)."""
    from memfast_amd import host_order

    capability = torch.backends.cpu.get_cpu_capability()
    print("torch CPU capability:", capability)
    assert host_order.sum_order_matches(), (
        f"torch CPU sum order on this host ({capability}) differs from the kernels' cascade")
    assert capability in host_order.VERIFIED_CAPABILITIES
    # The product's restatement agrees with this file's incremental one, column by column.
    values = host_order.probe_values()[0]
    np.testing.assert_array_equal(host_order.cascade_sum(values).numpy().view(np.int32),
                                  cascade_sum(values.numpy()).view(np.int32))


def test_order_probe_rejects_planted_orders():
    """A plain sequential sum and a cascade with another block size both differ from
    torch's sum on the probe values, so a host with either layout would be flagged."""
    from memfast_amd import host_order

    values = host_order.probe_values()[0]
    expected = values[None].sum(1)[0]
    sequential = torch.zeros(values.shape[1])
    for row in values:
        sequential = sequential + row
    assert not torch.equal(sequential, expected)
    blocks = [values[i:i + 8].sum(0) for i in range(0, values.shape[0], 8)]
    eights = torch.zeros(values.shape[1])
    for block in blocks:
        eights = eights + block
    assert not torch.equal(eights, expected)


@pytest.mark.parametrize("capability", ["avx2", "default"])
def test_order_does_not_depend_on_torch_cpu_capability(capability):
    """torch's CPU kernels forced to another vector ISA (ATEN_CPU_CAPABILITY, in a fresh
    process) reduce in the same order: FP32 and FP64 chunks with cascade and interleaved
    columns equal the kernels' order bit for bit."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    script = """
import sys
import torch
from memfast_amd import host_order
assert torch.backends.cpu.get_cpu_capability() == sys.argv[1].upper(), torch.backends.cpu.get_cpu_capability()
assert host_order.sum_order_matches()
for dtype, view in ((torch.float32, torch.int32), (torch.float64, torch.int64)):
    for reads in (3, 17, 64, 300):
        for columns in (4, 7, 24, 40, 72, 100):
            values = host_order.probe_values(reads=reads, columns=columns, dtype=dtype)
            got = host_order.kernel_order_sum(values[0])
            assert torch.equal(values.sum(1)[0].view(view), got.view(view)), (dtype, reads, columns)
print("ok", torch.backends.cpu.get_cpu_capability())
"""
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, ATEN_CPU_CAPABILITY=capability, PYTHONPATH=str(root))
    result = subprocess.run([sys.executable, "-c", script, capability], env=env,
                            capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stderr[-2000:]
    assert result.stdout.strip() == f"ok {capability.upper()}"


def test_product_model_matches_this_restatement_and_rejects_other_spans():
    """host_order.kernel_order_sum (the product's guard) equals this file's incremental
    restatement on FP32 chunks with interleaved columns; and an FP64 chunk classified with
    the FP32 span (32 instead of 16) differs from torch's sum."""
    from memfast_amd import host_order

    values = host_order.probe_values(reads=100, columns=72)[0]
    np.testing.assert_array_equal(host_order.kernel_order_sum(values).numpy().view(np.int32),
                                  kernel_sum(values.numpy()).view(np.int32))
    wide = host_order.probe_values(reads=100, columns=24, dtype=torch.float64)[0]
    expected = wide[None].sum(1)[0]
    assert torch.equal(host_order.kernel_order_sum(wide), expected)
    # With a 32-column span all 24 columns would be interleaved; the first 16 are not.
    assert not torch.equal(host_order.interleaved_sum(wide)[:16], expected[:16])
