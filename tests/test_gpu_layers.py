"""Drop-in layers on the GPU (memfast/nn: Linear, Conv2d, GRU, convert_model).

Each layer's output is compared with the CPU oracle applied the way the
reference composes it: AnalogLinear = one programmed matrix with its bias
(memfast/nn/linear.py), AnalogConv2d = F.unfold patches read through one
matrix per group (memfast/nn/convolution.py), AnalogGRU = per-step input and
hidden projections (read events 0, 1, ...) under PyTorch's gate equations
(memfast/nn/recurrent.py).  Ideal devices: bit-exact; write noise: flipped
codes at most 1e-4 of all codes, outputs without a flipped total within 1e-5
relative (``oracle.flips.check_noisy``).
"""

import math

import pytest
import torch
from torch import nn
from torch.nn import functional as F

from memfast_amd import Config, Nonidealities, Simulator, convert_model
from memfast_amd.nn import AnalogConv2d, AnalogGRU, AnalogLinear
from oracle import oracle
from parity import check_product, gru_step_parity

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
    assert kind == "ideal"
    assert torch.equal(got.view(torch.int32), expected.view(torch.int32)), (
        (got - expected).abs().max())


@pytest.mark.parametrize("kind", list(EFFECTS))
def test_analog_linear(hip_device, kind):
    cfg = config(kind)
    torch.manual_seed(3)
    source = nn.Linear(200, 70)
    sim = Simulator(cfg, device=hip_device)
    layer = AnalogLinear(source.to(hip_device), sim, name="linear")
    x = torch.randn(2, 5, 200)
    got = layer(x.to(hip_device))
    assert got.shape == (2, 5, 70)
    check_product(cfg, got, x, source.weight.T, hip_device, name="linear", bias=source.bias,
                  label=f"linear {kind}")


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
    side = (9 + 2 - 3) // 2 + 1
    assert got.shape == (2, 6, side, side)
    patches = F.unfold(x, 3, 1, 1, 2)
    size = 4 // groups * 9
    per_group = 6 // groups
    rows = got.flatten(2).transpose(1, 2)            # [N, L, out_channels]
    for g in range(groups):
        block = slice(g * per_group, (g + 1) * per_group)
        check_product(cfg, rows[:, :, block], patches[:, g * size:(g + 1) * size].transpose(1, 2),
                      source.weight[block].flatten(1).T, hip_device, name=f"conv.group{g}",
                      bias=source.bias[block], label=f"conv {kind} group {g}")


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
    assert torch.equal(hidden[0].view(torch.int32), output[-1].view(torch.int32))
    if kind == "ideal":
        # Whole-sequence check: gate math runs on the GPU here and on the CPU in the
        # oracle, so values agree up to the transcendental functions' last bits.
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
            h = (1 - update) * torch.tanh(inn + reset * hn) + update * h
            expected.append(h)
        torch.testing.assert_close(output.cpu(), torch.stack(expected), rtol=1e-5, atol=1e-6)
    # Step by step at each step's read events: every projection read flip-aware against
    # the oracle, the gates bit for bit on the GPU.
    gru_step_parity(layer.cells[0], source, x, output, hip_device, label=f"small gru {kind}")


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


# Implicit im2col: (N, C, H, W, groups, kernel, stride, padding, dilation).
CONV_GEOMETRIES = [
    (2, 4, 9, 9, 1, (3, 3), (2, 2), (1, 1), (1, 1)),
    (3, 6, 11, 7, 2, (3, 2), (1, 2), (2, 0), (1, 1)),
    (1, 8, 13, 13, 4, (3, 3), (1, 1), (2, 2), (2, 2)),
    (2, 3, 20, 17, 1, (1, 1), (2, 2), (0, 0), (1, 1)),
    (2, 16, 10, 10, 1, (5, 5), (1, 1), (2, 2), (1, 1)),
    (1, 3, 96, 96, 1, (7, 7), (2, 2), (3, 3), (1, 1)),
    (1, 5, 4, 6, 1, (4, 6), (3, 1), (0, 0), (1, 1)),
]
# (array_size, rows_per_read, input quantization): 48-row arrays pad K to a non-multiple of 64.
CONV_QUANT = [((64, 32), 32, g) for g in ("fixed", (1, None), (1, 32), (4, 64), (None, None),
                                           (3, None))]
CONV_QUANT += [((48, 32), 16, g) for g in ("fixed", (1, None), (1, 16), (4, 16))]


def _conv_case(geometry):
    n, c, h, w, groups, kernel, stride, padding, dilation = geometry
    out = [(e + 2 * p - d * (k - 1) - 1) // s + 1
           for e, p, d, k, s in zip((h, w), padding, dilation, kernel, stride)]
    return n, c, groups, kernel, stride, padding, dilation, out


@pytest.mark.parametrize("geometry", CONV_GEOMETRIES)
@pytest.mark.parametrize("quant", CONV_QUANT, ids=lambda q: f"{q[0][0]}-{q[2]}")
def test_conv_input_tiles_match_unfold(hip_device, geometry, quant):
    """mf_conv_input_tiles == input quantization of F.unfold's patch matrix, bit for bit,
    for every convolution group; small cases also against the oracle's quantizer."""
    from memfast_amd import hip
    n, c, groups, kernel, stride, padding, dilation, out = _conv_case(geometry)
    array, rows_per_read, gran = quant
    extra = dict(array_size=array, rows_per_read=rows_per_read)
    if gran != "fixed":
        extra["input_quant_gran"] = gran
    cfg = config("ideal", **extra)
    torch.manual_seed(31)
    x = torch.randn(n, c, *geometry[2:4]) * 3
    x[:, :, ::3, 1::2] *= 20.0     # scale outliers so groups differ
    patches = F.unfold(x, kernel, dilation, padding, stride)
    per_group = c // groups
    size = per_group * kernel[0] * kernel[1]
    xd = x.to(hip_device)
    for g in range(groups):
        flat = patches[:, g * size:(g + 1) * size].transpose(1, 2).reshape(-1, size)
        fixed = None
        if gran == "fixed":
            fixed = (torch.rand(1, size) * 0.1 + 0.01)
        geom = (g * per_group, per_group, kernel, stride, padding, dilation, out)
        status = hip.status_word(hip_device)
        q, xscale = hip.conv_input_tiles(
            xd, cfg, geom, None if fixed is None else fixed.to(hip_device), status=status)
        ref_q, ref_scale = hip.input_tiles(
            flat.to(hip_device), cfg, None if fixed is None else fixed.to(hip_device))
        torch.cuda.synchronize()
        assert int(status.item()) == 0
        assert torch.equal(q.cpu(), ref_q.cpu()), (geometry, gran, g)
        assert torch.equal(xscale.cpu().view(torch.int32), ref_scale.cpu().view(torch.int32))
        if flat.shape[0] * size <= 200_000:
            oq, oscale = oracle.input_tiles(flat, cfg, fixed)
            assert torch.equal(q.cpu(), oq)
            assert torch.equal(xscale.cpu().view(torch.int32), oscale.view(torch.int32))


@pytest.mark.parametrize("gran", ["fixed", (1, 32)])
def test_conv_input_tiles_flag_only_gathered_nonfinite(hip_device, gran):
    """A non-finite pixel that some patch reads sets STATUS_INPUT; one that stride skips
    (absent from F.unfold's patches as well) does not."""
    from memfast_amd import hip
    extra = {} if gran == "fixed" else dict(input_quant_gran=gran)
    cfg = config("ideal", **extra)
    x = torch.randn(1, 2, 8, 8)
    geom = (0, 2, (1, 1), (2, 2), (0, 0), (1, 1), (4, 4))
    fixed = torch.full((1, 2), 0.05, device=hip_device) if gran == "fixed" else None
    skipped = x.clone()
    skipped[0, 1, 3, 5] = float("nan")        # odd row: never on the stride-2 grid
    assert torch.isfinite(F.unfold(skipped, 1, 1, 0, 2)).all()
    read = x.clone()
    read[0, 0, 4, 2] = float("inf")
    for value, flagged in ((skipped, False), (read, True)):
        status = hip.status_word(hip_device)
        hip.conv_input_tiles(value.to(hip_device), cfg, geom, fixed, status=status)
        torch.cuda.synchronize()
        assert bool(int(status.item()) & hip.STATUS_INPUT) == flagged
        if flagged:
            with pytest.raises(ValueError, match="finite"):
                hip.conv_input_tiles(value.to(hip_device), cfg, geom, fixed)


@pytest.mark.parametrize("kind", list(EFFECTS))
@pytest.mark.parametrize("geometry", CONV_GEOMETRIES[:5])
@pytest.mark.parametrize("mode", ["zeros", "reflect", "circular"])
def test_conv_implicit_path_matches_unfold_path(hip_device, kind, geometry, mode):
    """AnalogConv2d's implicit-im2col forward equals reading F.unfold's patches through the
    same programmed matrices (same read events), bit for bit; fixed scales and padding
    modes too."""
    n, c, groups, kernel, stride, padding, dilation, out = _conv_case(geometry)
    if mode != "zeros" and max(padding) == 0:
        pytest.skip("padding modes only differ with padding")
    cfg = config(kind)
    torch.manual_seed(32)
    source = nn.Conv2d(c, 2 * groups, kernel, stride=stride, padding=padding, dilation=dilation,
                       groups=groups, padding_mode=mode).to(hip_device)
    sim = Simulator(cfg, device=hip_device)
    layer = AnalogConv2d(source, sim, name="conv")
    x = torch.randn(n, c, *geometry[2:4], device=hip_device)
    for fixed in (None, 0.04):
        for matrix in layer.matrices:
            matrix.set_input_scale(fixed)
            matrix.reset_read()
        got = layer(x)
        for matrix in layer.matrices:
            matrix.reset_read()
        source_x, unfold_padding = x, padding
        if mode != "zeros":
            ph, pw = padding
            source_x, unfold_padding = F.pad(x, (pw, pw, ph, ph), mode=mode), (0, 0)
        patches = F.unfold(source_x, kernel, dilation, unfold_padding, stride)
        size = c // groups * kernel[0] * kernel[1]
        parts = [matrix(patches[:, g * size:(g + 1) * size].transpose(1, 2))
                 for g, matrix in enumerate(layer.matrices)]
        expected = torch.cat(parts, dim=-1).transpose(1, 2).reshape(n, 2 * groups, *out)
        assert torch.equal(got.view(torch.int32), expected.view(torch.int32)), (geometry, fixed)
        assert all(matrix._event == 1 for matrix in layer.matrices)


@pytest.mark.parametrize("effects", [dict(write_variation=0.02),
                                     dict(write_variation=0.02, read_variation=0.01)])
@pytest.mark.parametrize("bidirectional", [False, True])
def test_gru_sequence_matches_per_step_cells(hip_device, effects, bidirectional):
    """AnalogGRU over a sequence (input projections read in one product when the read
    cannot depend on its event) equals stepping each cell, bit for bit, with the same
    read-event counts."""
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))), nonidealities=Nonidealities(**effects))
    torch.manual_seed(7)
    source = nn.GRU(40, 64, num_layers=2, bidirectional=bidirectional).to(hip_device)
    x = torch.randn(9, 3, 40, device=hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    stepped = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    output, hidden = layer(x)
    directions = 2 if bidirectional else 1
    sequence, finals = x, []
    for lay in range(2):
        outs = []
        for d in range(directions):
            cell = stepped.cells[lay * directions + d]
            h = torch.zeros(3, 64, device=hip_device)
            values = []
            for t in (reversed(range(9)) if d else range(9)):
                h = cell(sequence[t], h)
                values.append(h)
            if d:
                values.reverse()
            outs.append(torch.stack(values))
            finals.append(h)
        sequence = torch.cat(outs, dim=-1) if directions == 2 else outs[0]
    assert torch.equal(output.view(torch.int32), sequence.view(torch.int32))
    assert torch.equal(hidden.view(torch.int32), torch.stack(finals).view(torch.int32))
    for a, b in zip(layer.cells, stepped.cells):
        assert a.input._event == b.input._event == 9
        assert a.hidden._event == b.hidden._event == 9


def test_gru_nonfinite_input_raises_at_its_step(hip_device):
    """A non-finite input at step t raises as in per-step reading: both projections have
    then completed t reads."""
    cfg = config("write", input_quant_gran=(1, None))
    torch.manual_seed(8)
    source = nn.GRU(40, 64).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    x = torch.randn(6, 2, 40, device=hip_device)
    x[4, 1, 3] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        layer(x)
    cell = layer.cells[0]
    assert cell.input._event == 4 and cell.hidden._event == 4


def test_gru_hidden_read_failure_leaves_per_step_read_counts(hip_device):
    """A hidden read that fails at step 1 (its FP32 and FP64 results overflow FP32) raises
    as in per-step reading, after two input reads and one hidden read.  Every hidden weight
    is 3e38 and the input biases hold the update gate shut and the candidate at +1, so after
    step 0 every hidden unit is about 1 and each hidden sum is about 64 * 3e38."""
    cfg = config("write", input_quant_gran=(1, None))
    torch.manual_seed(9)
    source = nn.GRU(40, 64).to(hip_device)
    with torch.no_grad():
        source.weight_hh_l0.fill_(3e38)
        source.bias_ih_l0[64:128] = -30.0
        source.bias_ih_l0[128:] = 30.0
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    x = torch.randn(6, 2, 40, device=hip_device)
    with pytest.raises(FloatingPointError):
        layer(x)
    cell = layer.cells[0]
    assert cell.input._event == 2 and cell.hidden._event == 1


def test_gru_gates_kernel_matches_torch_ops(hip_device):
    """mf_gru_gates equals PyTorch's separate elementwise gate ops on the GPU, bit for bit."""
    from memfast_amd import hip
    torch.manual_seed(9)
    n, width = 67, 131
    inputs = torch.randn(n, 3 * width, device=hip_device) * 4
    hidden = torch.randn(n, 3 * width, device=hip_device) * 4
    hx = torch.randn(n, width, device=hip_device)
    inputs[0, :8] = torch.tensor([0.0, -0.0, 88.0, -88.0, 1e-30, -104.0, 30.0, -30.0])
    got = hip.gru_gates(inputs, hidden, hx)
    ir, iz, inn = inputs.chunk(3, dim=-1)
    hr, hz, hn = hidden.chunk(3, dim=-1)
    reset = torch.sigmoid(ir + hr)
    update = torch.sigmoid(iz + hz)
    expected = (1 - update) * torch.tanh(inn + reset * hn) + update * hx
    assert torch.equal(got.view(torch.int32), expected.view(torch.int32)), (
        (got != expected).sum().item(), (got - expected).abs().max().item())


def _step_cells(model, x, directions, layers, hidden_size):
    """Reference traversal: each cell called per step (per-step reads), as the reference."""
    sequence, finals = x, []
    batch = x.shape[1]
    for lay in range(layers):
        outs = []
        for d in range(directions):
            cell = model.cells[lay * directions + d]
            h = torch.zeros(batch, hidden_size, device=x.device, dtype=x.dtype)
            values = []
            for t in (reversed(range(x.shape[0])) if d else range(x.shape[0])):
                h = cell(sequence[t], h)
                values.append(h)
            if d:
                values.reverse()
            outs.append(torch.stack(values))
            finals.append(h)
        sequence = torch.cat(outs, dim=-1) if directions == 2 else outs[0]
    return sequence, torch.stack(finals)


@pytest.mark.parametrize("nonlinearity", ["tanh", "relu"])
@pytest.mark.parametrize("bidirectional", [False, True])
def test_rnn_sequence_matches_per_step_cells(hip_device, nonlinearity, bidirectional):
    """AnalogRNN over a sequence equals stepping its cells, bit for bit, with the same
    read-event counts (write noise: input projections read in one product)."""
    from memfast_amd.nn import AnalogRNN
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(10)
    source = nn.RNN(24, 48, num_layers=2, nonlinearity=nonlinearity,
                    bidirectional=bidirectional).to(hip_device)
    x = torch.randn(7, 5, 24, device=hip_device)
    layer = AnalogRNN(source, Simulator(cfg, device=hip_device), name="rnn")
    stepped = AnalogRNN(source, Simulator(cfg, device=hip_device), name="rnn")
    output, hidden = layer(x)
    directions = 2 if bidirectional else 1
    expected, finals = _step_cells(stepped, x, directions, 2, 48)
    assert torch.equal(output.view(torch.int32), expected.view(torch.int32))
    assert torch.equal(hidden.view(torch.int32), finals.view(torch.int32))
    for a, b in zip(layer.cells, stepped.cells):
        assert a.input._event == b.input._event == 7


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gru_half_precision_sequence_matches_per_step_cells(hip_device, dtype):
    """Half-precision sequences take PyTorch's gate ops; the sequence equals stepping the
    cells bit for bit."""
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(11)
    source = nn.GRU(40, 64).to(hip_device).to(dtype)
    x = torch.randn(6, 3, 40, device=hip_device, dtype=dtype)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    stepped = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    output, hidden = layer(x)
    expected, finals = _step_cells(stepped, x, 1, 1, 64)
    assert output.dtype == dtype
    assert torch.equal(output.view(torch.int16), expected.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_conv_half_precision_implicit_matches_unfold(hip_device, dtype):
    """Half-precision inputs: the implicit-im2col forward equals reading F.unfold's
    patches of the same tensor, bit for bit, and keeps the input dtype."""
    cfg = config("write")
    torch.manual_seed(12)
    source = nn.Conv2d(6, 8, 3, stride=1, padding=1).to(hip_device)
    layer = AnalogConv2d(source, Simulator(cfg, device=hip_device), name="conv")
    x = torch.randn(2, 6, 10, 10, device=hip_device).to(dtype)
    got = layer(x)
    layer.matrices[0].reset_read()
    patches = F.unfold(x, 3, 1, 1, 1)
    expected = layer.matrices[0](patches.transpose(1, 2)).transpose(1, 2).reshape(2, 8, 10, 10)
    assert got.dtype == dtype
    assert torch.equal(got.view(torch.int16), expected.view(torch.int16))


def _assert_same_traversal(layer, stepped, x, layers, hidden_size, bidirectional=False):
    directions = 2 if bidirectional else 1
    output, hidden = layer(x)
    expected, finals = _step_cells(stepped, x, directions, layers, hidden_size)
    assert torch.equal(output.view(torch.int32), expected.view(torch.int32))
    assert torch.equal(hidden.view(torch.int32), finals.view(torch.int32))
    for a, b in zip(layer.cells, stepped.cells):
        assert (a.input._event, a.hidden._event) == (b.input._event, b.hidden._event)


def test_rnn_hidden_overflow_recovered_by_fp64_retry(hip_device):
    """ReLU hidden states near 2e36 make every hidden read from step 1 on overflow in its
    FP32 restore ((T * xs) * ws), while the FP64 retry gives sums near 5e25.  The deferred
    hidden reads flag this; the traversal then reads per step with the retry, exactly as
    stepping the cells does."""
    from memfast_amd.nn import AnalogRNN
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(13)
    source = nn.RNN(8, 16, nonlinearity="relu").to(hip_device)
    with torch.no_grad():
        source.weight_ih_l0.fill_(3e35)
        source.weight_hh_l0.uniform_(1e-12, 2e-12)
    x = torch.rand(5, 2, 8, device=hip_device) * 0.5 + 0.5
    layer = AnalogRNN(source, Simulator(cfg, device=hip_device), name="rnn")
    stepped = AnalogRNN(source, Simulator(cfg, device=hip_device), name="rnn")
    _assert_same_traversal(layer, stepped, x, 1, 16)
    output, _ = stepped(x)
    assert bool(torch.isfinite(output).all()) and output.abs().max() > 1e35


def test_gru_without_bias_sequence_matches_per_step_cells(hip_device):
    """bias=False: both projections are programmed without bias; the sequence equals
    stepping the cells."""
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(14)
    source = nn.GRU(40, 64, num_layers=2, bias=False).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    stepped = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    assert all(cell.input.bias is None and cell.hidden.bias is None for cell in layer.cells)
    _assert_same_traversal(layer, stepped, torch.randn(7, 3, 40, device=hip_device), 2, 64)


def test_gru_config3_shape_sequence_matches_per_step_cells(hip_device):
    """BASELINE config 3's shapes (input 40, hidden 512, batch 32) over 12 steps: the
    single input read and the deferred hidden reads equal stepping the cell."""
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
                 weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=7,
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(15)
    source = nn.GRU(40, 512).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    stepped = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    _assert_same_traversal(layer, stepped, torch.randn(12, 32, 40, device=hip_device), 1, 512)


def test_gru_hooks_see_every_step(hip_device):
    """Hooks on a cell or its projections see one call per step: with hooks present
    the traversal calls the cell at every step, as the reference does."""
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(16)
    source = nn.GRU(40, 64).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    plain = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    calls = {"cell": 0, "input": 0, "hidden": 0}

    def counter(key):
        def hook(module, args, output):
            calls[key] += 1
        return hook

    cell = layer.cells[0]
    handles = [cell.register_forward_hook(counter("cell")),
               cell.input.register_forward_hook(counter("input")),
               cell.hidden.register_forward_hook(counter("hidden"))]
    x = torch.randn(6, 3, 40, device=hip_device)
    output, _ = layer(x)
    assert calls == {"cell": 6, "input": 6, "hidden": 6}
    expected, _ = plain(x)
    assert torch.equal(output.view(torch.int32), expected.view(torch.int32))
    for handle in handles:
        handle.remove()
    layer(x)
    assert calls == {"cell": 6, "input": 6, "hidden": 6}


def test_gru_gate_failure_sets_per_step_read_counts(hip_device, monkeypatch):
    """Steps queued from Python: a failure after step 2's hidden read (forced from the host
    in the gate call) leaves both projections at three reads, as per-step reading would."""
    from memfast_amd.nn import recurrent
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(17)
    source = nn.GRU(40, 64).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    monkeypatch.setattr(recurrent, "_native_eligible", lambda *args: False)
    gates = recurrent.hip.gru_gates
    count = {"calls": 0}

    def failing(*args):
        count["calls"] += 1
        if count["calls"] == 3:
            raise RuntimeError("forced gate failure")
        return gates(*args)

    monkeypatch.setattr(recurrent.hip, "gru_gates", failing)
    with pytest.raises(RuntimeError, match="forced gate failure"):
        layer(torch.randn(6, 3, 40, device=hip_device))
    cell = layer.cells[0]
    assert (cell.input._event, cell.hidden._event) == (3, 3)


def test_gru_native_sequence_failure_counts_one_input_read(hip_device, monkeypatch):
    """A failing native sequence call (forced from the host) fails as step 0's hidden read
    would: one input read, no hidden read."""
    from memfast_amd.nn import recurrent
    cfg = Config(**(BASE | dict(input_quant_gran=(1, None))),
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(18)
    source = nn.GRU(40, 64).to(hip_device)
    layer = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    x = torch.randn(6, 3, 40, device=hip_device)
    assert recurrent._native_eligible(layer.cells[0], torch.empty(6, 3, 192, device=hip_device),
                                      torch.zeros(3, 64, device=hip_device), 6)

    def failing(*args, **kwargs):
        raise RuntimeError("forced sequence failure")

    monkeypatch.setattr(recurrent.hip, "gru_sequence", failing)
    with pytest.raises(RuntimeError, match="forced sequence failure"):
        layer(x)
    cell = layer.cells[0]
    assert (cell.input._event, cell.hidden._event) == (1, 0)


@pytest.mark.parametrize("kind", ["ideal", "write"])
@pytest.mark.parametrize("bidirectional", [False, True])
def test_gru_native_and_python_steps_agree(hip_device, kind, bidirectional, monkeypatch):
    """The native sequence call (ideal: k_ideal, write noise: k_noisy) equals the steps
    queued from Python, bit for bit, with the same read counts."""
    from memfast_amd.nn import recurrent
    cfg = config(kind, input_quant_gran=(1, None))
    torch.manual_seed(19)
    source = nn.GRU(40, 96, num_layers=2, bidirectional=bidirectional).to(hip_device)
    x = torch.randn(8, 5, 40, device=hip_device)
    native = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    python = AnalogGRU(source, Simulator(cfg, device=hip_device), name="gru")
    assert recurrent._native_eligible(native.cells[0], torch.empty(8, 5, 288, device=hip_device),
                                      torch.zeros(5, 96, device=hip_device), 8)
    got, got_h = native(x)
    with monkeypatch.context() as patch:
        patch.setattr(recurrent, "_native_eligible", lambda *args: False)
        expected, expected_h = python(x)
    assert torch.equal(got.view(torch.int32), expected.view(torch.int32))
    assert torch.equal(got_h.view(torch.int32), expected_h.view(torch.int32))
    for a, b in zip(native.cells, python.cells):
        assert (a.input._event, a.hidden._event) == (b.input._event, b.hidden._event) == (8, 8)


WIDE_CONV = {
    # BFP16 activations, INT4 weights (BASELINE config 5's slicing) on 64x64 arrays
    "bfp16": dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                  weight_slice=(1, 1, 2), bw_e=8, array_size=(64, 64), adc_bits=(6, 6, 7)),
    # 12-bit INT activations, 32-row reads, groups of 64 columns
    "int12": dict(activation_bits=12, weight_bits=8, input_slice=(1, 3, 4, 4),
                  weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                  adc_bits=8, input_quant_gran=(1, 64)),
}


@pytest.mark.parametrize("name", list(WIDE_CONV))
@pytest.mark.parametrize("geometry", CONV_GEOMETRIES[:5])
def test_wide_conv_input_tiles_match_unfold(hip_device, name, geometry):
    """mf_conv_input_tiles_wide == wide input quantization of F.unfold's patch matrix
    (uint32 codes, FP64 scales), bit for bit, dynamic and fixed scales; small cases also
    against the oracle's quantizer."""
    from memfast_amd import hip
    n, c, groups, kernel, stride, padding, dilation, out = _conv_case(geometry)
    cfg = Config(**WIDE_CONV[name], nonidealities=Nonidealities(write_variation=0.0))
    torch.manual_seed(33)
    x = torch.randn(n, c, *geometry[2:4]) * 3
    x[:, :, ::3, 1::2] *= 20.0
    patches = F.unfold(x, kernel, dilation, padding, stride)
    per_group = c // groups
    size = per_group * kernel[0] * kernel[1]
    xd = x.to(hip_device)
    for g in range(groups):
        flat = patches[:, g * size:(g + 1) * size].transpose(1, 2).reshape(-1, size)
        geom = (g * per_group, per_group, kernel, stride, padding, dilation, out)
        for fixed in (None, torch.rand(1, size, dtype=torch.float64) * 0.1 + 0.01):
            fixed_dev = None if fixed is None else fixed.to(hip_device)
            status = hip.status_word(hip_device)
            q, xscale = hip.conv_input_tiles(xd, cfg, geom, fixed_dev, status=status)
            ref_q, ref_scale = hip.input_tiles(flat.to(hip_device), cfg, fixed_dev)
            assert int(status.item()) == 0
            assert q.dtype == torch.int32 and xscale.dtype == torch.float64
            assert torch.equal(q.cpu(), ref_q.cpu()), (name, geometry, g, fixed is None)
            assert torch.equal(xscale.cpu().view(torch.int64), ref_scale.cpu().view(torch.int64))
            if fixed is None and flat.shape[0] * size <= 100_000:
                oq, oscale = oracle.input_tiles(flat, cfg)
                assert torch.equal(q.cpu().to(oq.dtype), oq)
                assert torch.equal(xscale.cpu().view(torch.int64), oscale.view(torch.int64))


@pytest.mark.parametrize("case", ["wide_default", "narrow_tuned", "wide_tuned"])
def test_conv_gathered_forward_matches_unfold_in_wide_and_tuned_modes(hip_device, case,
                                                                      tmp_path):
    """The gathered forward of wide configurations and of tuned mode equals reading
    F.unfold's patches through the same matrices (same read events), bit for bit."""
    wide = case.startswith("wide")
    mode = "tuned" if case.endswith("tuned") else "default"
    kwargs = WIDE_CONV["int12"] if wide else BASE
    cfg = Config(**kwargs, nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(34)
    source = nn.Conv2d(6, 8, 3, stride=1, padding=1, groups=2).to(hip_device)
    sim = Simulator(cfg, device=hip_device, mode=mode, cache_dir=tmp_path)
    layer = AnalogConv2d(source, sim, name="conv")
    x = torch.randn(2, 6, 9, 9, device=hip_device)
    got = layer(x)
    assert all(matrix._event == 1 for matrix in layer.matrices)
    for matrix in layer.matrices:
        matrix.reset_read()
    expected = torch.cat(layer._unfolded(x, (1, 1)), dim=-1).transpose(1, 2).reshape(2, 8, 9, 9)
    view = torch.int64 if got.dtype == torch.float64 else torch.int32
    assert got.dtype == torch.float32
    assert torch.equal(got.view(view), expected.view(view))
    if mode == "tuned":
        assert len(sim.records) >= 2


def test_conv_tuned_nonfinite_input_raises_before_search(hip_device, tmp_path):
    """Tuned mode: a non-finite pixel raises the read's error before any schedule is
    searched or cached."""
    cfg = config("write")
    source = nn.Conv2d(4, 4, 3, padding=1).to(hip_device)
    sim = Simulator(cfg, device=hip_device, mode="tuned", cache_dir=tmp_path)
    layer = AnalogConv2d(source, sim, name="conv")
    x = torch.randn(1, 4, 6, 6, device=hip_device)
    x[0, 2, 3, 3] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        layer(x)
    assert not sim.records and layer.matrices[0]._event == 0
    assert not any(tmp_path.rglob("*.json"))
