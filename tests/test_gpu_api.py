"""The Python API around the hot path, on the GPU: functional mm/matmul, the trainable
``nn.Linear``/``nn.Conv2d`` layers, hardware-aware training and ``convert_model``.

Forward values are compared bit for bit with the oracle (ideal devices).  Gradients
follow the reference's quantized-operand surrogate (memfast/nn/training.py:55-93,
memfast/functional.py:130-136): dx uses the dequantized grouped weights, dw the
dequantized grouped inputs; the expected values are built on the CPU from the
oracle's own quantizer and compared to 1e-5 (both sides are FP32 BLAS products in
different summation orders).  Selection semantics of ``convert_model`` follow
memfast/nn/conversion.py:26-243 and docs/user-guide.md:55-81.
"""

import copy
import dataclasses
import math

import pytest
import torch
from torch import nn
from torch.nn import functional as F

import memfast_amd as memfast
from memfast_amd import Config, Nonidealities, Simulator, convert_model
from memfast_amd import nn as analog_nn
from memfast_amd.nn import AnalogConv2d, AnalogGRU, AnalogLinear, reset_read_events
from oracle import oracle

pytestmark = pytest.mark.gpu

IDEAL = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
               weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
               weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8),
               nonidealities=Nonidealities(write_variation=0.0))


def bits_equal(a, b):
    a, b = a.detach().cpu(), b.detach().cpu().to(a.dtype)
    view = {torch.float32: torch.int32, torch.float64: torch.int64,
            torch.float16: torch.int16, torch.bfloat16: torch.int16}[a.dtype]
    return a.shape == b.shape and torch.equal(a.view(view), b.view(view))


def dequantized(value, bits, granularity, cfg, signed=True):
    code, scale = oracle.grouped_quantize(value.detach().cpu(), bits, granularity, cfg.bw_e,
                                          signed=signed)
    return (code * scale).float()


def surrogate_grads(a, b, grad, cfg):
    """(dA, dB) of the reference's quantized-operand surrogate of a @ b (a [N,K], b [K,O])."""
    a_dq = dequantized(a, cfg.activation_bits, cfg.input_quant_gran, cfg)
    b_dq = dequantized(b, cfg.weight_bits, cfg.weight_quant_gran, cfg, cfg.weight_signed)
    return grad.cpu() @ b_dq.T, a_dq.T @ grad.cpu()


def close(got, expected, label=""):
    expected = expected.to(torch.float64)
    scale = expected.abs().max().item()
    torch.testing.assert_close(got.detach().cpu().double(), expected, rtol=1e-5,
                               atol=1e-6 * max(scale, 1e-30), msg=label)


# ---------------------------------------------------------------------------
# functional mm / matmul
# ---------------------------------------------------------------------------
def test_mm_forward_and_surrogate_gradients(hip_device):
    gen = torch.Generator().manual_seed(81)
    a = torch.randn(20, 150, generator=gen)
    b = torch.randn(150, 40, generator=gen)
    grad = torch.randn(20, 40, generator=gen)
    ad = a.to(hip_device).requires_grad_()
    bd = b.to(hip_device).requires_grad_()
    out = memfast.mm(ad, bd, config=IDEAL)
    assert bits_equal(out, oracle.mm(a, b, IDEAL))
    out.backward(grad.to(hip_device))
    da, db = surrogate_grads(a, b, grad, IDEAL)
    close(ad.grad, da, "dA")
    close(bd.grad, db, "dB")
    # Without gradients requested no surrogate is attached.
    plain = memfast.mm(a.to(hip_device), b.to(hip_device), config=IDEAL)
    assert not plain.requires_grad and bits_equal(plain, out)


MATMUL_SHAPES = [((150,), (150, 40)), ((7, 150), (150,)), ((3, 7, 150), (150, 40)),
                 ((150,), (4, 150, 40)), ((2, 1, 5, 150), (3, 150, 40)),
                 ((3, 5, 150), (3, 150, 40))]


@pytest.mark.parametrize("left,right", MATMUL_SHAPES, ids=[f"{l}@{r}" for l, r in MATMUL_SHAPES])
def test_matmul_shapes_and_programs(hip_device, left, right):
    """torch.matmul shapes; one program per distinct right-hand matrix; with per-row input
    groups and ideal devices every output row equals a separate read of its operands."""
    gen = torch.Generator().manual_seed(82)
    a = torch.randn(left, generator=gen)
    b = torch.randn(right, generator=gen)
    cfg = Config(activation_bits=8, weight_bits=8, array_size=(64, 32), adc_bits=8,
                 input_quant_gran=(1, None), nonidealities=Nonidealities(write_variation=0.0))
    sim = Simulator(cfg, device=hip_device)
    got = sim.matmul(a.to(hip_device), b.to(hip_device))
    assert got.shape == torch.matmul(a, b).shape
    b2 = b if b.ndim > 1 else b[:, None]
    rhs_batch = b2.shape[:-2]
    assert sim._next_id == max(1, math.prod(rhs_batch))
    # Row-by-row reference: broadcast both operands to the batch, read each RHS matrix.
    a2 = a if a.ndim > 1 else a[None]
    batch = torch.broadcast_shapes(a2.shape[:-2], b2.shape[:-2])
    a3 = a2.expand(*batch, *a2.shape[-2:]).reshape(-1, *a2.shape[-2:])
    b3 = b2.expand(*batch, *b2.shape[-2:]).reshape(-1, *b2.shape[-2:])
    expected = torch.stack([oracle.mm(a3[i], b3[i], cfg) for i in range(a3.shape[0])])
    assert bits_equal(got.reshape(-1), expected.reshape(-1))


@pytest.mark.parametrize("route", ["simulator", "functional"])
def test_rhs_program_names_follow_tensor_geometry(hip_device, route):
    """A rank-two RHS is its own program key (memfast/simulator.py:133-171): after an
    in-place change of its geometry the new program takes over the old one's name and
    read-event counter.  A vector RHS is read through a view of its tensor
    (memfast/functional.py:95-127), so the same tensor with a new geometry is a new RHS.
    Simulator.mm's direct route and the general functional route agree."""
    cfg = dataclasses.replace(
        IDEAL, nonidealities=Nonidealities(write_variation=0.02, read_variation=0.01))
    sim = Simulator(cfg, device=hip_device)
    gen = torch.Generator().manual_seed(83)
    a = torch.randn(6, 150, generator=gen).to(hip_device)
    b = torch.randn(150, 40, generator=gen).to(hip_device)
    mm = sim.mm if route == "simulator" else (lambda x, y: memfast.mm(x, y, simulator=sim))
    first, second = mm(a, b), mm(a, b)
    program = sim._matrix_cache.program(b)
    assert (program.name, program._event, sim._next_id) == ("matrix.0", 2, 1)
    b.data = b.data.T.contiguous().T          # same values, new strides
    assert b.stride() != (40, 1)
    third = mm(a, b)
    program = sim._matrix_cache.program(b)
    assert (program.name, program._event, sim._next_id) == ("matrix.0", 3, 1)
    # The reads used name matrix.0 at events 0, 1, 2, as a fresh simulator's reads do.
    fresh, same = Simulator(cfg, device=hip_device), b.contiguous()
    reads = [fresh.mm(a, same) for _ in range(3)]
    assert all(bits_equal(got, want) for got, want in zip((first, second, third), reads))
    assert not bits_equal(reads[1], reads[2])   # read noise follows the event
    # Vector RHS: a new geometry of the same tensor is a new RHS with a new name.
    v = torch.randn(150, generator=gen).to(hip_device)
    sim.matmul(a, v)
    key = sim._next_id
    v.data = torch.randn(300, generator=gen).to(hip_device)[::2]
    sim.matmul(a, v)
    assert sim._next_id == key + 1


def test_mm_out_and_argument_errors(hip_device):
    a = torch.randn(4, 64, device=hip_device)
    b = torch.randn(64, 8, device=hip_device)
    out = torch.empty(4, 8, device=hip_device)
    result = memfast.mm(a, b, config=IDEAL, out=out)
    assert result is out and bits_equal(out, memfast.mm(a, b, config=IDEAL))
    with pytest.raises(ValueError, match="out must have the result shape"):
        memfast.mm(a, b, config=IDEAL, out=torch.empty(4, 9, device=hip_device))
    with pytest.raises(RuntimeError, match="out= does not support"):
        memfast.mm(a.clone().requires_grad_(), b, config=IDEAL, out=out)
    with pytest.raises(ValueError, match="incompatible reduction"):
        memfast.mm(a, b[:60], config=IDEAL)
    with pytest.raises(ValueError, match="same dtype"):
        memfast.mm(a, b.double(), config=IDEAL)
    with pytest.raises(ValueError, match="rank-two"):
        memfast.mm(a[0], b, config=IDEAL)
    with pytest.raises(TypeError, match="real floating dense"):
        memfast.mm(a.int(), b.int(), config=IDEAL)
    with pytest.raises(ValueError, match="batch dimensions cannot broadcast"):
        memfast.matmul(torch.randn(2, 4, 64, device=hip_device),
                       torch.randn(3, 64, 8, device=hip_device), config=IDEAL)
    sim = Simulator(IDEAL, device=hip_device)
    with pytest.raises(ValueError, match="config differs"):
        memfast.mm(a, b, simulator=sim, config=Config())
    empty = memfast.mm(a[:0], b, config=IDEAL)
    assert empty.shape == (0, 8)


# ---------------------------------------------------------------------------
# nn.Linear / nn.Conv2d (trainable, PyTorch signatures)
# ---------------------------------------------------------------------------
def test_nn_linear_programming_training_and_state(hip_device):
    torch.manual_seed(83)
    layer = analog_nn.Linear(150, 40, config=IDEAL, device=hip_device)
    assert set(layer.state_dict()) == {"weight", "bias"}
    assert isinstance(layer.weight, nn.Parameter) and layer.weight.shape == (40, 150)
    x = torch.randn(6, 150)
    grad = torch.randn(6, 40)
    xd = x.to(hip_device).requires_grad_()
    out = layer(xd)
    w, bias = layer.weight.detach().cpu(), layer.bias.detach().cpu()
    q, xs = oracle.input_tiles(x, IDEAL)
    packed, ws = oracle.weight_tiles(w, IDEAL)
    seed = oracle.name_seed(IDEAL.seed, layer.matrix.name)
    assert bits_equal(out, oracle.execute(q, xs, packed, ws, IDEAL, seed, 0, 40, bias=bias))
    out.backward(grad.to(hip_device))
    dx, dwt = surrogate_grads(x, w.T, grad, IDEAL)
    close(xd.grad, dx, "dx")
    close(layer.weight.grad, dwt.T, "dW")
    close(layer.bias.grad, grad.sum(0), "db")
    # An optimizer step is picked up by the next forward (reprogramming).
    optimizer = torch.optim.SGD(layer.parameters(), lr=0.5)
    optimizer.step()
    after = layer(x.to(hip_device))
    w2, b2 = layer.weight.detach().cpu(), layer.bias.detach().cpu()
    packed, ws = oracle.weight_tiles(w2, IDEAL)
    assert bits_equal(after, oracle.execute(q, xs, packed, ws, IDEAL, seed, 1, 40, bias=b2))
    # update_weight copies PyTorch-layout weights without replacing the Parameter.
    parameter = layer.weight
    new = torch.randn(40, 150)
    layer.update_weight(new.to(hip_device))
    assert layer.weight is parameter and torch.equal(layer.weight.detach().cpu(), new)
    with pytest.raises(ValueError, match="original PyTorch shape"):
        layer.update_weight(torch.randn(40, 151, device=hip_device))
    # State dicts carry PyTorch names only; loading reprograms.
    other = analog_nn.Linear(150, 40, config=IDEAL, device=hip_device)
    other.load_state_dict(layer.state_dict())
    assert bits_equal(other(x.to(hip_device)), layer(x.to(hip_device)))


def test_nn_conv2d_padding_groups_and_gradients(hip_device):
    torch.manual_seed(84)
    conv = analog_nn.Conv2d(4, 6, 3, padding="same", groups=2, config=IDEAL, device=hip_device)
    assert set(conv.state_dict()) == {"weight", "bias"}
    x = torch.randn(2, 4, 7, 7)
    xd = x.to(hip_device).requires_grad_()
    out = conv(xd)
    assert out.shape == (2, 6, 7, 7)
    w, bias = conv.weight.detach().cpu(), conv.bias.detach().cpu()
    patches = F.unfold(F.pad(x, (1, 1, 1, 1)), 3)
    parts = []
    for g, matrix in enumerate(conv.analog.matrices):
        flat = patches[:, g * 18:(g + 1) * 18].transpose(1, 2).reshape(-1, 18)
        q, xs = oracle.input_tiles(flat, IDEAL)
        parts.append(oracle.execute(q, xs, *oracle.weight_tiles(w[3 * g:3 * g + 3].flatten(1),
                                                                IDEAL),
                                    IDEAL, 0, 0, 3, bias=bias[3 * g:3 * g + 3]).reshape(2, 49, 3))
    expected = torch.cat(parts, -1).transpose(1, 2).reshape(2, 6, 7, 7)
    assert bits_equal(out, expected)
    grad = torch.randn(2, 6, 7, 7)
    out.backward(grad.to(hip_device))
    # dx through the dequantized-weight surrogate on unfolded patches, folded back.
    xf = x.clone().requires_grad_()
    pieces = []
    pf = F.unfold(F.pad(xf, (1, 1, 1, 1)), 3)
    for g in range(2):
        cols = pf[:, g * 18:(g + 1) * 18].transpose(1, 2).reshape(-1, 18)
        xq = dequantized(cols, 8, IDEAL.input_quant_gran, IDEAL)
        operand = cols + (xq - cols).detach()
        wq = dequantized(w[3 * g:3 * g + 3].flatten(1).T, 8, IDEAL.weight_quant_gran, IDEAL)
        pieces.append((operand @ wq).reshape(2, 49, 3))
    surrogate = torch.cat(pieces, -1).transpose(1, 2).reshape(2, 6, 7, 7)
    surrogate.backward(grad)
    close(xd.grad, xf.grad, "dx")
    assert conv.weight.grad is not None and conv.bias.grad is not None
    close(conv.bias.grad, grad.sum((0, 2, 3)), "db")
    # Unbatched input follows nn.Conv2d.
    assert conv(x[0].to(hip_device)).shape == (6, 7, 7)


@pytest.mark.parametrize("mode", ["quantized", "digital"])
def test_convert_model_training_shares_parameters(hip_device, mode):
    torch.manual_seed(85)
    model = nn.Sequential(nn.Linear(100, 30), nn.Tanh(), nn.Linear(30, 5)).to(hip_device)
    trainable = convert_model(model, Simulator(IDEAL, device=hip_device), training=True,
                              gradient_mode=mode)
    assert trainable.training
    layer = trainable[0]
    assert type(layer).__name__ == "TrainableAnalogLinear" and layer.gradient_mode == mode
    x = torch.randn(8, 100, device=hip_device, requires_grad=True)
    y = trainable(x)
    y.sum().backward()
    w = layer.weight.detach().cpu()
    hidden_grad = (1 - torch.tanh(trainable[0](x.detach()).cpu()) ** 2)
    assert layer.weight.grad is not None and x.grad is not None
    if mode == "digital":
        # dx of the unquantized digital layers (through the analog tanh values).
        w2 = trainable[2].weight.detach().cpu()
        expected = (hidden_grad * w2.sum(0)) @ w
        close(x.grad, expected, "digital dx")
    # The trained parameters are the converted copy's own, not the source model's.
    assert layer.weight is not model[0].weight
    with pytest.raises(ValueError, match="gradient_mode"):
        convert_model(model, Simulator(IDEAL, device=hip_device), training=True,
                      gradient_mode="exact")


# ---------------------------------------------------------------------------
# convert_model selection semantics
# ---------------------------------------------------------------------------
class _Net(nn.Module):
    def __init__(self):
        super().__init__()
        self.stem = nn.Conv2d(3, 4, 3, padding=1)
        self.body = nn.Sequential(nn.Linear(8, 8), nn.ReLU(), nn.Linear(8, 8))
        self.head = nn.Linear(8, 2)
        self.shared = nn.Linear(8, 8)
        self.block = nn.Sequential(self.shared)    # second alias of `shared`
        self.rnn = nn.GRU(8, 8)


def kinds(model):
    """Layer type by path, leaving out the projections inside converted recurrent layers."""
    return {name: type(module).__name__ for name, module in model.named_modules()
            if isinstance(module, (nn.Linear, nn.Conv2d, nn.GRU, AnalogLinear, AnalogConv2d,
                                   AnalogGRU)) and ".cells." not in name}


def test_convert_model_selection_rules(hip_device):
    sim = Simulator(IDEAL, device=hip_device)
    net = _Net()
    everything = convert_model(net, sim)
    assert kinds(everything) == {"stem": "AnalogConv2d", "body.0": "AnalogLinear",
                                 "body.2": "AnalogLinear", "head": "AnalogLinear",
                                 "shared": "AnalogLinear", "rnn": "AnalogGRU"}
    assert everything.shared is everything.block[0]          # one replacement per module
    assert not everything.training and not any(p.requires_grad for p in everything.parameters())
    assert type(net.head) is nn.Linear                       # the source model is untouched
    assert kinds(convert_model(net, sim, include=())) == kinds(net)
    subset = convert_model(net, sim, include=["body"], exclude=["body.2"])
    assert kinds(subset)["body.0"] == "AnalogLinear" and kinds(subset)["body.2"] == "Linear"
    assert kinds(subset)["head"] == "Linear"
    root = convert_model(net, sim, include=[""], exclude=["rnn"])
    assert kinds(root)["rnn"] == "GRU" and kinds(root)["stem"] == "AnalogConv2d"
    # A shared module converts only when every alias is included and none excluded.
    one_alias = convert_model(net, sim, include=["shared", "head"])
    assert type(one_alias.shared) is nn.Linear and type(one_alias.head) is AnalogLinear
    both = convert_model(net, sim, include=["shared", "block"])
    assert type(both.shared) is AnalogLinear and both.block[0] is both.shared
    excluded_alias = convert_model(net, sim, exclude=["block"])
    assert type(excluded_alias.shared) is nn.Linear
    # Names of converted layers are their module paths (they seed the noise samples).
    assert everything.head.name == "head" and everything.stem.matrices[0].name == "stem.group0"
    assert everything.rnn.cells[0].input.name.startswith("rnn")
    # In place conversion edits and returns the model itself.
    target = _Net()
    assert convert_model(target, sim, inplace=True) is target
    assert type(target.head) is AnalogLinear


def test_convert_model_argument_errors(hip_device):
    sim = Simulator(IDEAL, device=hip_device)
    net = _Net()
    with pytest.raises(ValueError, match=r"unknown included modules: \['nope'\]"):
        convert_model(net, sim, include=["nope"])
    with pytest.raises(ValueError, match=r"unknown excluded modules"):
        convert_model(net, sim, exclude=["head.x"])
    with pytest.raises(TypeError, match="sequence of module paths"):
        convert_model(net, sim, include="head")
    with pytest.raises(TypeError, match="module paths must be strings"):
        convert_model(net, sim, exclude=[3])
    with pytest.raises(TypeError, match="PyTorch module"):
        convert_model(object(), sim)
    with pytest.raises(TypeError, match="training must be a boolean"):
        convert_model(net, sim, training=1)
    same = nn.Sequential(nn.Conv2d(3, 4, 3, padding="same"))
    with pytest.raises(ValueError, match="numeric Conv2d padding"):
        convert_model(same, sim)
    converted = convert_model(net, sim)
    with pytest.raises(ValueError, match="selection inside a converted layer"):
        convert_model(converted, sim, include=["stem.matrices.0"])
    other = Simulator(Config(activation_bits=8, weight_bits=8, array_size=(64, 32), adc_bits=7),
                      device=hip_device)
    with pytest.raises(ValueError, match="matching physical config and mode"):
        convert_model(converted, other)
    with pytest.raises(ValueError, match="original digital layer weights"):
        convert_model(converted, sim, training=True)
    # Reconversion with the same simulator keeps the programmed layers.
    again = convert_model(converted, sim)
    assert torch.equal(again.head.packed, converted.head.packed)


def test_convert_model_llama_partitions_and_read_events(hip_device):
    class Cfg:
        model_type, pretraining_tp = "llama", 4

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.config = Cfg()
            self.proj = nn.Linear(8, 8)

    sim = Simulator(Config(activation_bits=8, weight_bits=8, array_size=(64, 32), adc_bits=8,
                           nonidealities=Nonidealities(write_variation=0.02, read_variation=0.02)),
                    device=hip_device)
    block = Block()
    converted = convert_model(block, sim)
    assert converted.config.pretraining_tp == 1 and block.config.pretraining_tp == 4
    x = torch.randn(3, 8, device=hip_device)
    first = converted.proj(x)
    converted.proj(x)
    assert converted.proj._event == 2
    reset_read_events(converted)
    assert converted.proj._event == 0
    assert bits_equal(converted.proj(x), first)
    assert copy.deepcopy(converted).proj._event == 1
