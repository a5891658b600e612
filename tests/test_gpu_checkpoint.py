"""The reference's own static LeNet-5 checkpoint, loaded into a converted network.

examples/checkpoints/lenet5_mnist_static_int4.pt (written by the reference's
examples/04_lenet5_mnist_static_quant.py:128-185) holds, for each of LeNet-5's
five analog matrices, packed INT4 codes, weight scales, fixed input scales,
biases and ``_extra_state`` (config, name, seed, read event).  Its tensors and
extra states are in tests/golden/lenet_int4.npz (tests/golden/make_lenet_fixture.py).

The test converts a locally defined LeNet-5 with the example's Config, loads
that state with ``load_state_dict(strict=True)`` (memfast/simulator.py:452-534,
memfast/nn/modules.py:45-72), checks the state round trip, and checks every
analog layer's read of a fixed batch against the oracle applied to the
checkpoint's own codes, scales, biases, seeds and events: bit for bit with
ideal devices, under the flip accounting with the checkpoint's write variation.
Each layer is fed the GPU network's own input to it, so that one layer's
rounding flips do not carry into the next layer's comparison.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from memfast_amd import AnalogMatrix, Config, Nonidealities, Simulator, convert_model
from memfast_amd.nn import AnalogConv2d, AnalogLinear
from netdefs import LeNet5
from oracle import oracle
from parity import check_read, gpu_totals, say

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).with_name("golden") / "lenet_int4.npz"


def fixture():
    return np.load(FIXTURE, allow_pickle=False)


def example_config(write_variation):
    """The example's simulator Config (examples/04_lenet5_mnist_static_quant.py:40-52)."""
    return Config(activation_bits=8, weight_bits=4, input_slice=None, weight_slice=None,
                  array_size=(64, 64), rows_per_read=None, input_quant_gran=(1, None),
                  weight_quant_gran=(None, 1), adc_bits=6, bw_e=None,
                  nonidealities=Nonidealities(write_variation=write_variation))


def checkpoint_state(write_variation=None, edit=None):
    """The checkpoint's state dict; ``write_variation`` rewrites the saved configs' write
    variation (a checkpoint written with that device model), ``edit(state)`` plants a
    mistake."""
    data = fixture()
    state = {}
    for index in range(int(data["count"])):
        prefix = str(data[f"l{index}_prefix"])
        for name in ("packed", "weight_scale", "input_scale", "bias"):
            state[f"{prefix}.{name}"] = torch.from_numpy(data[f"l{index}_{name}"].copy())
        extra = json.loads(str(data[f"l{index}_extra_state"]))
        if write_variation is not None:
            extra["config"]["nonidealities"]["write_variation"] = write_variation
        state[f"{prefix}._extra_state"] = extra
    assert sorted(state) == sorted(str(k) for k in data["state_keys"])
    if edit is not None:
        edit(state)
    return state


def converted(cfg, device):
    torch.manual_seed(0)
    model = LeNet5().float()
    saved = json.loads(str(fixture()["conversion"]))
    return convert_model(model, Simulator(cfg, device=device), include=saved["include"],
                         exclude=tuple(saved["exclude"]))


@pytest.mark.parametrize("write_variation", [0.0, 0.02])
def test_static_checkpoint_loads_and_reads_like_the_reference(hip_device, write_variation):
    cfg = example_config(write_variation)
    state = checkpoint_state(None if write_variation == 0.02 else write_variation)
    model = converted(cfg, hip_device)
    model.load_state_dict(state, strict=True)

    # Round trip: the model's state is the checkpoint's.
    saved = model.state_dict()
    assert sorted(saved) == sorted(state)
    for key, value in state.items():
        if key.endswith("_extra_state"):
            mine = saved[key]
            assert (mine["name"], mine["seed"], mine["event"]) == (
                value["name"], value["seed"], value["event"])
            assert json.loads(json.dumps(mine["config"])) == value["config"] | dict(
                nonidealities={k: v for k, v in value["config"]["nonidealities"].items()
                               if k != "output_noise"})
        else:
            assert torch.equal(saved[key].cpu(), value), key

    # One fixed batch; capture each analog layer's input and output.
    layers = {name: module for name, module in model.named_modules()
              if isinstance(module, (AnalogConv2d, AnalogLinear))}
    assert sorted(layers) == ["classifier.0", "classifier.2", "classifier.4", "features.0",
                              "features.3"]
    seen = {}
    hooks = [module.register_forward_hook(
        lambda module, inputs, output, name=name: seen.__setitem__(name, (inputs[0], output)))
        for name, module in layers.items()]
    gen = torch.Generator().manual_seed(17)
    images = torch.rand(8, 1, 28, 28, generator=gen) * 2 - 1     # Normalize((0.5,), (0.5,))
    logits = model(images.to(hip_device))
    for hook in hooks:
        hook.remove()
    assert logits.shape == (8, 10) and torch.isfinite(logits).all()

    for name, module in layers.items():
        inputs, output = seen[name]
        matrix = module.matrices[0] if isinstance(module, AnalogConv2d) else module
        prefix = f"{name}.matrices.0" if isinstance(module, AnalogConv2d) else name
        extra = state[f"{prefix}._extra_state"]
        assert (matrix.name, matrix.seed, matrix._event) == (extra["name"], extra["seed"], 1)
        if isinstance(module, AnalogConv2d):
            patches = F.unfold(inputs.cpu(), module.kernel_size, module.dilation, module.padding,
                               module.stride)
            flat = patches.transpose(1, 2).reshape(-1, patches.shape[1])
            got = output.flatten(2).transpose(1, 2).reshape(-1, module.out_channels)
        else:
            flat, got = inputs.cpu(), output
        q, xs = oracle.input_tiles(flat, cfg, state[f"{prefix}.input_scale"])
        packed, ws = state[f"{prefix}.packed"], state[f"{prefix}.weight_scale"]
        bias = state[f"{prefix}.bias"]
        out_features = bias.shape[0]
        if write_variation == 0.0:
            expected = oracle.execute(q, xs, packed, ws, cfg, extra["seed"], extra["event"],
                                      out_features, bias=bias)
            assert torch.equal(got.cpu().view(torch.int32), expected.view(torch.int32)), name
            say(name, "bit-exact")
        else:
            totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, extra["seed"],
                                extra["event"])
            check_read(cfg, got, q, xs, packed, ws, extra["seed"], extra["event"], totals,
                       bias=bias, label=f"lenet {name}")


def _set(key, value):
    def edit(state):
        state[key] = value
    return edit


def _config_edit(path, value):
    def edit(state):
        extra = state["classifier.2._extra_state"]
        target = extra["config"]
        for part in path[:-1]:
            target = target[part]
        target[path[-1]] = value
    return edit


REJECTED = {
    "float codes": (_set("classifier.0.packed", torch.zeros(7, 2, 64, 64)),
                    "integer dtype"),
    "codes beyond 4 bits": (_set("classifier.0.packed", torch.full((7, 2, 64, 64), 16,
                                                                     dtype=torch.uint8)),
                            "exceed the configured bit width"),
    "negative scale": (_set("classifier.4.weight_scale", -torch.ones(2, 1, 64)),
                       "finite and nonnegative"),
    "infinite scale": (_set("classifier.4.weight_scale", torch.full((2, 1, 64), float("inf"))),
                       "finite and nonnegative"),
    "other ADC": (_config_edit(("adc_bits",), 7), "physical configuration differs"),
    "removed noise model": (_config_edit(("nonidealities", "output_noise"), 0.1),
                            "removed noise model"),
    "seed beyond 32 bits": (lambda state: state["classifier.2._extra_state"].__setitem__(
        "seed", 2**32), "sampling seed"),
    "other matrix width": (lambda state: state["classifier.2._extra_state"].__setitem__(
        "out_features", 85), "logical matrix dimensions"),
}


@pytest.mark.parametrize("case", list(REJECTED))
def test_static_checkpoint_validation(hip_device, case):
    """Checkpoint validation of memfast/simulator.py:452-534 (dtype, range, finiteness,
    physical configuration, removed noise model, seed, matrix dimensions)."""
    edit, message = REJECTED[case]
    model = converted(example_config(0.02), hip_device)
    with pytest.raises(ValueError, match=message):
        model.load_state_dict(checkpoint_state(edit=edit), strict=True)


def test_checkpoint_read_events_replay(hip_device):
    """A loaded program continues from the checkpoint's read event; reset_read replays it."""
    from memfast_amd.nn import reset_read_events

    cfg = Config(**dict(activation_bits=8, weight_bits=8, array_size=(64, 64), adc_bits=8),
                 nonidealities=Nonidealities(write_variation=0.02, read_variation=0.02))
    torch.manual_seed(3)
    source = torch.nn.Linear(100, 30)
    first = convert_model(torch.nn.Sequential(source), Simulator(cfg, device=hip_device))
    x = torch.randn(4, 100, device=hip_device)
    reads = [first(x) for _ in range(3)]
    state = first.state_dict()
    assert state["0._extra_state"]["event"] == 3
    second = convert_model(torch.nn.Sequential(torch.nn.Linear(100, 30)),
                           Simulator(cfg, device=hip_device))
    second.load_state_dict(state)
    assert isinstance(second[0], AnalogMatrix) and second[0]._event == 3
    reset_read_events(second, 1)
    again = second(x)
    assert torch.equal(again.view(torch.int32), reads[1].view(torch.int32))
