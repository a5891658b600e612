"""mf_mm_static, the read that allocates nothing, against mf_mm through the C-ABI.

mf_mm_static takes the scratch mf_mm gets as a workspace from the library's
static device array instead.  Its outputs must equal mf_mm's bit for bit (the
same kernels and noise samples), on two calls in a row with the second one
smaller, for an ideal-device read (digit masks in the array) and for a noisy
read whose conductance terms exceed the array (read in column chunks there,
while mf_mm reads the whole program at once from its own workspace).  A read
whose scratch cannot fit fails with MF_E_RESOURCE before any launch.
"""

import ctypes as ct

import pytest
import torch

from memfast_amd import Config, Nonidealities, hip

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 64 << 20     # MF_STATIC_SCRATCH_BYTES (include/memfast_hip.h)

INT8 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
            weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))
CASES = {
    "ideal": (Nonidealities(write_variation=0.0), [(300, 1024, 700), (70, 384, 200)], 1),
    # 1024 x 4096 programs hold 84 MB of conductance terms: beyond the 64 MiB array.
    "noisy": (Nonidealities(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1),
              [(256, 1024, 4096), (64, 512, 300)], 2),
}


def say(*args):
    print("[no-alloc]", *args, flush=True)


def _operands(cfg, n, k, o, device, seed):
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(n, k, generator=gen).to(device)
    b = torch.randn(k, o, generator=gen).to(device)
    q, xscale = hip.input_tiles(a, cfg)
    packed, packed_t, wscale = hip.weight_tiles(b.T, cfg)
    return q, xscale, packed, packed_t, wscale


def mm_static(q, xscale, packed, packed_t, wscale, cfg, seed, event, out_cols, k_rows):
    n, m, _ = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    out = torch.full((n, p * c), float("nan"), device=q.device)
    status = hip.status_word(q.device)
    rc = hip.library().mf_mm_static(
        ct.byref(hip.descriptor(cfg)), hip._ptr(q), hip._ptr(xscale), n, m, hip._ptr(packed),
        hip._ptr(packed_t), hip._ptr(wscale.reshape(-1, p * c)), p, out_cols, k_rows, None,
        seed, event, hip._ptr(out), out.stride(0), 0, hip._ptr(status), hip._stream(q.device))
    hip.check(rc, "mm static")
    return out, status


@pytest.mark.parametrize("kind", list(CASES))
def test_static_scratch_read_equals_mm(hip_device, kind):
    effects, shapes, kernel = CASES[kind]
    cfg = Config(**INT8, nonidealities=effects)
    for call, (n, k, o) in enumerate(shapes):
        say(kind, "call", call, (n, k, o))
        q, xscale, packed, packed_t, wscale = _operands(cfg, n, k, o, hip_device, 10 + call)
        m, p = q.shape[1], packed.shape[1]
        assert hip.mm_kernel(cfg, n, m, p) == kernel
        if kind == "noisy" and call == 0:   # the chunked path inside the array
            assert hip.mm_workspace_bytes(cfg, n, m, p) > STATIC_SCRATCH_BYTES
        seed, event = 1000 + call, 3 + call
        expected_status = hip.status_word(hip_device)
        expected = hip.mm(q, xscale, packed, packed_t, wscale.reshape(-1, p * cfg.array_size[1]),
                          cfg, seed, event, status=expected_status, out_cols=o, k_rows=k)
        got, status = mm_static(q, xscale, packed, packed_t, wscale, cfg, seed, event, o, k)
        torch.cuda.synchronize()
        assert int(status.item()) == int(expected_status.item()) == 0
        assert torch.equal(got[:, :o].view(torch.int32), expected[:, :o].view(torch.int32)), (
            kind, call, int((got[:, :o] != expected[:, :o]).sum()))


def test_static_scratch_rejects_reads_beyond_it(hip_device):
    """Binary weights on 128-row arrays at K = 40960: one 64-column chunk of conductance
    terms (256*W*m*R = 84 MB) exceeds the 64 MiB array, so the call fails before any
    launch."""
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=None, array_size=(128, 128), rows_per_read=32, adc_bits=8,
                 nonidealities=Nonidealities(write_variation=0.02))
    q, xscale, packed, packed_t, wscale = _operands(cfg, 64, 40960, 64, hip_device, 7)
    assert hip.mm_kernel(cfg, 64, q.shape[1], packed.shape[1]) == 2
    with pytest.raises(hip.ResourceError, match="MF_STATIC_SCRATCH_BYTES"):
        mm_static(q, xscale, packed, packed_t, wscale, cfg, 5, 0, 64, 40960)
