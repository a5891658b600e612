"""Drop-in layers on the GPU (memfast/nn: Linear, Conv2d, GRU, convert_model).

Each layer's output is compared with the CPU oracle applied the way the
reference composes it: AnalogLinear = one programmed matrix with its bias
(memfast/nn/linear.py), AnalogConv2d = F.unfold patches read through one
matrix per group (memfast/nn/convolution.py), AnalogGRU = per-step input and
hidden projections (read events 0, 1, ...) under PyTorch's gate equations
(memfast/nn/recurrent.py).  Ideal devices: bit-exact; write noise: within
the rounding-flip budget.
"""

import math

import pytest
import torch
from torch import nn
from torch.nn import functional as F

from memfast_amd import Config, Nonidealities, Simulator, convert_model
from memfast_amd.nn import AnalogConv2d, AnalogGRU, AnalogLinear
from oracle import oracle

pytestmark = pytest.mark.gpu

BASE = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
            weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))
EFFECTS = {"ideal": dict(write_variation=0.0), "write": dict(write_variation=0.02)}


def config(kind, **extra):
    return Config(**(BASE | extra), nonidealities=Nonidealities(**EFFECTS[kind]))


def oracle_matrix(x, weight, bias, cfg, name, event=0):
    """One AnalogMatrix read of x [..., K] with PyTorch [O, K] weights, on the CPU."""
    x = x.detach().cpu()
    flat = x.reshape(-1, weight.shape[1])
    packed, wscale = oracle.weight_tiles(weight.detach().cpu(), cfg)
    q, xscale = oracle.input_tiles(flat, cfg)
    seed = oracle.name_seed(cfg.seed, name)
    out = oracle.execute(q, xscale, packed, wscale, cfg, seed, event, weight.shape[0],
                         bias=None if bias is None else bias.detach().cpu().float())
    return out.reshape(*x.shape[:-1], weight.shape[0]).to(x.dtype)


def check(got, expected, kind):
    got = got.detach().cpu()
    if kind == "ideal":
        assert torch.equal(got.view(torch.int32), expected.view(torch.int32)), (
            (got - expected).abs().max())
    else:
        rel = (got - expected).abs() / expected.abs().clamp_min(1e-6)
        assert (rel > 1e-5).float().mean().item() <= 0.02


@pytest.mark.parametrize("kind", list(EFFECTS))
def test_analog_linear(hip_device, kind):
    cfg = config(kind)
    torch.manual_seed(3)
    source = nn.Linear(200, 70)
    sim = Simulator(cfg, device=hip_device)
    layer = AnalogLinear(source.to(hip_device), sim, name="linear")
    x = torch.randn(2, 5, 200)
    got = layer(x.to(hip_device))
    check(got, oracle_matrix(x, source.weight, source.bias, cfg, "linear"), kind)


@pytest.mark.parametrize("kind", list(EFFECTS))
@pytest.mark.parametrize("groups", [1, 2])
def test_analog_conv2d(hip_device, kind, groups):
    cfg = config(kind)
    torch.manual_seed(4)
    source = nn.Conv2d(4, 6, 3, stride=2, padding=1, groups=groups)
    sim = Simulator(cfg, device=hip_device)
    layer = AnalogConv2d(source.to(hip_device), sim, name="conv")
    x = torch.randn(2, 4, 9, 9)
    got = layer(x.to(hip_device))
    patches = F.unfold(x, 3, 1, 1, 2)
    size = 4 // groups * 9
    per_group = 6 // groups
    parts = []
    for g in range(groups):
        block = slice(g * per_group, (g + 1) * per_group)
        parts.append(oracle_matrix(patches[:, g * size:(g + 1) * size].transpose(1, 2),
                                   source.weight[block].flatten(1), source.bias[block], cfg,
                                   f"conv.group{g}"))
    side = (9 + 2 - 3) // 2 + 1
    expected = torch.cat(parts, dim=-1).transpose(1, 2).reshape(2, 6, side, side)
    check(got, expected, kind)


@pytest.mark.parametrize("kind", list(EFFECTS))
def test_analog_gru(hip_device, kind):
    """Config-3 shape in miniature: 1-layer GRU, per-step analog projections."""
    cfg = config(kind)
    torch.manual_seed(5)
    source = nn.GRU(40, 64, num_layers=1)
    sim = Simulator(cfg, device=hip_device)
    layer = AnalogGRU(source.to(hip_device), sim, name="gru")
    steps, batch = 6, 3
    x = torch.randn(steps, batch, 40)
    output, hidden = layer(x.to(hip_device))
    h = torch.zeros(batch, 64)
    expected = []
    for t in range(steps):
        inputs = oracle_matrix(x[t], source.weight_ih_l0, source.bias_ih_l0, cfg,
                               "gru.layer0.direction0.input", event=t)
        hid = oracle_matrix(h, source.weight_hh_l0, source.bias_hh_l0, cfg,
                            "gru.layer0.direction0.hidden", event=t)
        ir, iz, inn = inputs.chunk(3, dim=-1)
        hr, hz, hn = hid.chunk(3, dim=-1)
        reset = torch.sigmoid(ir + hr)
        update = torch.sigmoid(iz + hz)
        candidate = torch.tanh(inn + reset * hn)
        h = (1 - update) * candidate + update * h
        expected.append(h)
    expected = torch.stack(expected)
    if kind == "ideal":
        # Gate math runs on the GPU here and on the CPU in the oracle: same values up to
        # the transcendental functions' last bits.
        torch.testing.assert_close(output.cpu(), expected, rtol=1e-5, atol=1e-6)
    else:
        assert (output.cpu() - expected).abs().max().item() <= 1e-3
    torch.testing.assert_close(hidden[0].cpu(), output[-1].cpu())


def test_convert_model(hip_device):
    """convert_model replaces Conv2d/Linear with analog layers; outputs compose as oracle reads."""
    cfg = config("ideal")
    torch.manual_seed(6)
    model = nn.Sequential(nn.Conv2d(3, 4, 3, padding=1), nn.ReLU(), nn.Flatten(),
                          nn.Linear(4 * 6 * 6, 10)).eval()
    sim = Simulator(cfg, device=hip_device)
    converted = convert_model(model.to(hip_device), sim)
    assert isinstance(converted[0], AnalogConv2d) and isinstance(converted[3], AnalogLinear)
    x = torch.randn(2, 3, 6, 6)
    got = converted(x.to(hip_device)).cpu()
    conv, linear = model[0].cpu(), model[3].cpu()
    patches = F.unfold(x, 3, 1, 1, 1)
    hidden = oracle_matrix(patches.transpose(1, 2), conv.weight.flatten(1), conv.bias, cfg,
                           "0.group0")
    hidden = F.relu(hidden.transpose(1, 2).reshape(2, 4, 6, 6)).flatten(1)
    expected = oracle_matrix(hidden, linear.weight, linear.bias, cfg, "3")
    check(got, expected, "ideal")
    assert math.isfinite(got.abs().max().item())
