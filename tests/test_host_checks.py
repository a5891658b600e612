"""Host-side logic of the layer read's early status check (no GPU): the cached maxima of
the fixed scales and bias, and the bound that decides whether a read can leave a
non-finite FP32 output."""
from types import SimpleNamespace

import torch

from memfast_amd import Config
from memfast_amd.simulator import AnalogMatrix


def _stub(config, input_scale=0.05, weight_scale=0.01, bias=0.5, mode="default",
          zero_correction=None):
    return SimpleNamespace(
        simulator=SimpleNamespace(mode=mode), config=config,
        input_scale=None if input_scale is None else torch.full((1, 300), input_scale),
        weight_scale=torch.full((5, 90), weight_scale),
        bias=None if bias is None else torch.full((90,), bias),
        zero_correction=zero_correction)


def _bounded(stub, arrays=5):
    stub._host_max = lambda name, tensor: AnalogMatrix._host_max(stub, name, tensor)
    return AnalogMatrix._output_bounded(stub, arrays)


def test_host_max_follows_tensor_identity_and_version():
    stub = SimpleNamespace()
    t = torch.tensor([1.0, -3.0])
    assert AnalogMatrix._host_max(stub, "s", t) == 3.0
    t.mul_(2.0)   # in place: a new version
    assert AnalogMatrix._host_max(stub, "s", t) == 6.0
    other = t.view(2)   # another tensor object over the same storage
    other.data.fill_(7.0)   # (.data writes do not count as versions of `t`)
    assert AnalogMatrix._host_max(stub, "s", other) == 7.0
    replaced = torch.tensor([0.25])
    assert AnalogMatrix._host_max(stub, "s", replaced) == 0.25


def test_output_bound_cases():
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), adc_bits=6)
    assert _bounded(_stub(cfg))
    assert not _bounded(_stub(cfg, input_scale=None))            # dynamic scales
    assert not _bounded(_stub(cfg, mode="tuned"))
    assert not _bounded(_stub(cfg, zero_correction=torch.zeros(1)))
    assert not _bounded(_stub(cfg, bias=torch.finfo(torch.float32).max))
    assert not _bounded(_stub(cfg, input_scale=1e37))
    # The bound itself: G reads * reconstruction_bound * xs * ws * 1.07 + |b| < FLT_MAX / 2.
    reads = 5 * cfg.reads_per_array
    edge = torch.finfo(torch.float32).max / 2 / (reads * cfg.reconstruction_bound * 0.01 * 1.07)
    assert _bounded(_stub(cfg, input_scale=edge * 0.99, bias=None))
    assert not _bounded(_stub(cfg, input_scale=edge * 1.01, bias=None))
    bfp = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                 weight_slice=(1, 1, 2), bw_e=8, array_size=(64, 64), adc_bits=(6, 6, 7))
    assert not _bounded(_stub(bfp))
