"""Imported integer weights: ``Simulator.map_quantized`` with and without zero points
(memfast/simulator.py:173-185 programming, :587-611 digital zero-point correction).

The programmed buffers (packed codes, per-read scales, correction rows) equal the
oracle's bit for bit, and so does the analog read itself.  The zero-point term is
``(sum of signed input codes per read * input scale) @ zero_correction``, a BLAS
matrix product over the G reads in the reference, evaluated by torch on the GPU here
and on the CPU in the oracle; their summation orders differ, so outputs with zero
points are held to 1e-5 relative (plus 1e-6 of the largest correction term), which
still catches a dropped or mis-signed correction by orders of magnitude.
"""

import pytest
import torch

from memfast_amd import Config, Nonidealities, Simulator
from oracle import oracle

pytestmark = pytest.mark.gpu

CASES = {
    # unsigned 4-bit codes (weight_signed=False), per-channel scales and zero points
    "unsigned_int4": dict(activation_bits=8, weight_bits=4, weight_signed=False,
                          input_slice=(1, 1, 2, 2, 2), weight_slice=(2, 2), array_size=(64, 32),
                          rows_per_read=32, adc_bits=8, input_quant_gran=(1, 32)),
    # signed 8-bit codes on 128x128 arrays (BASELINE config 2's slicing)
    "signed_int8": dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                        weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
                        adc_bits=(6, 7, 7, 8, 8), input_quant_gran=(1, 32)),
    # 12-bit activations: FP64 restore and the per-chunk FP64 correction
    "wide_int12": dict(activation_bits=12, weight_bits=4, weight_signed=False,
                       input_slice=(1, 1, 2, 2, 2, 2, 2), weight_slice=(2, 2),
                       array_size=(64, 32), rows_per_read=32, adc_bits=8,
                       input_quant_gran=(1, 32)),
}


def bits_equal(a, b):
    a, b = a.detach().cpu(), b.detach().cpu().to(a.dtype)
    view = torch.int32 if a.dtype == torch.float32 else torch.int64
    return a.shape == b.shape and torch.equal(a.view(view), b.view(view))


@pytest.mark.parametrize("case", list(CASES))
def test_map_quantized_matches_oracle(hip_device, case):
    cfg = Config(**CASES[case], nonidealities=Nonidealities(write_variation=0.0))
    gen = torch.Generator().manual_seed(71)
    o, k, n = 70, 300, 9
    if cfg.weight_signed:
        codes = torch.randint(-127, 128, (o, k), generator=gen)
        zero_points = torch.randint(-20, 21, (o, 1), generator=gen).float()
    else:
        codes = torch.randint(0, 16, (o, k), generator=gen)
        zero_points = torch.randint(2, 14, (o, 1), generator=gen).float()
    scales = torch.rand(o, 1, generator=gen) * 0.05 + 0.01
    bias = torch.randn(o, generator=gen)
    x = torch.randn(n, k, generator=gen)

    packed, wscale, correction = oracle.imported_tiles(codes, scales, cfg, zero_points)
    q, xs = oracle.input_tiles(x, cfg)
    seed0, seed1 = oracle.name_seed(cfg.seed, "matrix.0"), oracle.name_seed(cfg.seed, "matrix.1")

    sim = Simulator(cfg, device=hip_device)
    plain = sim.map_quantized(codes.to(hip_device), scales.to(hip_device), bias=bias.to(hip_device))
    affine = sim.map_quantized(codes.to(hip_device), scales.to(hip_device),
                               zero_points=zero_points.to(hip_device), bias=bias.to(hip_device))
    assert bits_equal(plain.packed, packed) and bits_equal(plain.weight_scale, wscale)
    assert plain.zero_correction is None
    assert bits_equal(affine.zero_correction, correction)

    # Without zero points the whole read, bias included, is bit-exact.
    expected = oracle.execute(q, xs, packed, wscale, cfg, seed0, 0, o, bias=bias.to(xs.dtype))
    assert bits_equal(plain(x.to(hip_device)), expected.float())

    got = affine(x.to(hip_device)).cpu().double()
    expected = oracle.execute(q, xs, packed, wscale, cfg, seed1, 0, o, bias=bias.to(xs.dtype),
                              zero_correction=correction).double()
    uncorrected = oracle.execute(q, xs, packed, wscale, cfg, seed1, 0, o,
                                 bias=bias.to(xs.dtype)).double()
    scale = (expected - uncorrected).abs().max().item()
    torch.testing.assert_close(got, expected, rtol=1e-5, atol=1e-6 * scale)
    assert (uncorrected - expected).abs().max().item() > 1e3 * (got - expected).abs().max().item()
