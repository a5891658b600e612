"""GPU parity at BASELINE's own configurations.

Each test runs the configuration's ``Config`` as written in BASELINE.json and
compares against the CPU oracle:
  * config 1, the README product with write variation;
  * config 2's noisy leg (write 0.02, shared read 0.01, S-curve 0.1) on
    128x128 arrays: injected conductances on a K=4096 row sample, sampled
    conductances through a full 4096^3 Simulator.mm, and a full-size row
    permutation property;
  * config 3, the converted GRU (40 -> 512, batch 32) for eight steps;
  * config 4, ResNet-18's 7x7/2 stem and a 3x3 64->64 convolution at batch 2,
    plus a full-size batch-64 batch-permutation property of the whole network.

Noisy reads follow BASELINE's bar through ``oracle.flips.check_noisy``: flipped
codes (counted from the slice totals behind each output) at most 1e-4 of all
codes, every output whose totals all match within 1e-5 relative, and every
other output within the effect of its own flips.
"""

import pytest
import torch
from torch import nn
from torch.nn import functional as F

from memfast_amd import Config, Nonidealities, Simulator, convert_model, hip
from memfast_amd.nn import AnalogConv2d, reset_read_events
from oracle import flips, oracle
from netdefs import resnet18
from parity import check_read, gpu_totals, gru_step_parity, say

pytestmark = pytest.mark.gpu

INT8 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2))
CONFIG2 = INT8 | dict(array_size=(128, 128), rows_per_read=32, weight_quant_gran=(32, 1),
                      input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))
CONFIG2_NOISY = Nonidealities(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1)


def bits_equal(a, b):
    a, b = a.detach().cpu().contiguous(), b.detach().cpu().contiguous()
    view = torch.int32 if a.dtype == torch.float32 else torch.int64
    return a.shape == b.shape and torch.equal(a.view(view), b.view(view))


# ---------------------------------------------------------------------------
# Config 1: README first simulation, 4x128 @ 128x32, ADC 7, write variation 0.02
# ---------------------------------------------------------------------------
def test_config1_write_noise(hip_device):
    cfg = Config(**INT8, array_size=(128, 128), rows_per_read=32, weight_quant_gran=(32, 1),
                 input_quant_gran=(1, 32), adc_bits=7,
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(135)
    a, b = torch.randn(4, 128), torch.randn(128, 32)
    got = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, 0)
    check_read(cfg, got, q, xs, packed, ws, seed, 0, totals, label="config1")


# ---------------------------------------------------------------------------
# Config 2, noisy leg: 128x128 arrays, 32-row reads, ADC (6,7,7,8,8)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def config2_operands():
    torch.manual_seed(135)
    return torch.randn(4096, 4096), torch.randn(4096, 4096)


def test_config2_noisy_injected_conductances(hip_device, config2_operands):
    """The MFMA read's slice totals equal the oracle's given the oracle's own sampled
    conductances (all 4096 rows of K, two tiles of columns), except rounding flips."""
    cfg = Config(**CONFIG2, nonidealities=CONFIG2_NOISY)
    a, b = config2_operands
    rows = torch.tensor([0, 5, 1000, 2047, 3001, 4095])
    q, _ = oracle.input_tiles(a[rows], cfg)
    packed, _ = oracle.weight_tiles(b[:, 512:768].T, cfg)
    n, m, _ = q.shape
    assert hip.mm_kernel(cfg, 4096, m, 32) == 2
    seed, event = oracle.name_seed(cfg.seed, "matrix.0"), 3
    raw, _, _ = oracle.restored(packed, cfg, seed, event, 0, packed.shape[1])
    expected = oracle.partial(q, packed, cfg, seed, event, 0, packed.shape[1], conductance=raw)
    got = hip.mm_totals(q.to(hip_device), hip.kernel_codes(packed.to(hip_device), cfg), cfg,
                        seed, event, conductance=raw.to(hip_device))
    differing, flipped, unexplained, mask = flips.count_flips(cfg, got, expected)
    codes = mask.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    say("config2 injected:", differing, "differing totals,", flipped, "flips of", codes, "codes")
    assert unexplained == 0
    assert flipped <= max(1, 1e-4 * codes)


@pytest.fixture(scope="module")
def config2_noisy_output(hip_device, config2_operands):
    cfg = Config(**CONFIG2, nonidealities=CONFIG2_NOISY)
    a, b = config2_operands
    say("config2 noisy 4096^3 Simulator.mm")
    out = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    torch.cuda.synchronize()
    return cfg, out


def test_config2_noisy_full_size_rows(hip_device, config2_operands, config2_noisy_output):
    """Full 4096^3 Simulator.mm with GPU-sampled conductances: a row sample against the
    oracle (its own samples) in the first and last two-tile chunks."""
    cfg, out = config2_noisy_output
    a, b = config2_operands
    rows = torch.tensor([0, 1, 777, 2048, 4095])
    q, xs = oracle.input_tiles(a[rows], cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, 0)
    got = out[rows.to(hip_device)].cpu()
    for first in (0, 30):
        tiles = (first, first + 2)
        check_read(cfg, got[:, first * 128:(first + 2) * 128], q, xs, packed, ws, seed, 0,
                   totals, tiles=tiles, label=f"config2 rows, tiles {tiles}")


def test_config2_noisy_full_size_row_permutation(hip_device, config2_operands,
                                                 config2_noisy_output):
    """Every noise sample is keyed by cell address and read event, and input groups are
    per row: permuting A's rows permutes the 4096^3 output's rows, bit for bit."""
    cfg, out = config2_noisy_output
    a, b = config2_operands
    perm = torch.randperm(4096, generator=torch.Generator().manual_seed(2))
    permuted = Simulator(cfg, device=hip_device).mm(a[perm].to(hip_device), b.to(hip_device))
    assert bits_equal(permuted, out[perm.to(hip_device)])
    assert not bits_equal(permuted, out)


# ---------------------------------------------------------------------------
# Config 3: converted GRU 40 -> 512, batch 32, ADC 7, write variation 0.02
# ---------------------------------------------------------------------------
def test_config3_gru_steps(hip_device):
    """Eight steps of BASELINE config 3's converted GRU.  Per step: the layer's output is
    PyTorch's gate equations over the two projection reads at that step's read event
    (bit for bit on the GPU, within transcendental rounding on the CPU), and each read
    matches the oracle under the flip accounting."""
    cfg = Config(**INT8, array_size=(128, 128), rows_per_read=32, adc_bits=7,
                 nonidealities=Nonidealities(write_variation=0.02))
    torch.manual_seed(135)
    source = nn.GRU(40, 512, 1)
    steps, batch = 8, 32
    x = torch.randn(steps, batch, 40)
    layer = convert_model(source.to(hip_device), Simulator(cfg, device=hip_device))
    output, hidden = layer(x.to(hip_device))
    assert bits_equal(hidden[0], output[-1])
    cell = layer.cells[0]
    assert hip.mm_kernel(cfg, batch, 4, cell.hidden.p) == 2
    gru_step_parity(cell, source, x, output, hip_device, label="config3")


# ---------------------------------------------------------------------------
# Config 4: ResNet-18 on 256x256 arrays, 64-row reads, per-output-channel weight
# groups, fixed input scales, ADC 8, write variation 0.02 + 0.1% stuck-at faults
# ---------------------------------------------------------------------------
CONFIG4 = Config(**INT8, array_size=(256, 256), rows_per_read=64, weight_quant_gran=(None, 1),
                 adc_bits=8, nonidealities=Nonidealities(write_variation=0.02,
                                                         stuck_at_low=0.0005,
                                                         stuck_at_high=0.0005))
CONV_LAYERS = {   # Conv2d arguments (in, out, kernel, stride, padding), input shape
    "stem_7x7_s2": ((3, 64, 7, 2, 3), (2, 3, 224, 224)),
    "layer1_3x3": ((64, 64, 3, 1, 1), (2, 64, 56, 56)),
}


@pytest.mark.parametrize("name", list(CONV_LAYERS))
def test_config4_convolution(hip_device, name):
    """One ResNet-18 convolution at batch 2 with a calibrated fixed input scale: a sample
    of 512 patch rows (fixed scales quantize element-wise, so any row subset quantizes
    alike) against the oracle reading F.unfold's patches (memfast/nn/convolution.py:49-54)."""
    torch.manual_seed(135)
    arguments, shape = CONV_LAYERS[name]
    source = nn.Conv2d(*arguments, bias=False)
    nn.init.kaiming_normal_(source.weight, mode="fan_out", nonlinearity="relu")
    calibration = max(float(torch.randn(shape).abs().amax()) for _ in range(4))
    scale = calibration / 127
    x = torch.randn(shape)
    layer = AnalogConv2d(source.to(hip_device), Simulator(CONFIG4, device=hip_device),
                         name=name)
    matrix = layer.matrices[0]
    matrix.set_input_scale(scale)
    got = layer(x.to(hip_device))
    patches = F.unfold(x, source.kernel_size, source.dilation, source.padding, source.stride)
    flat = patches.transpose(1, 2).reshape(-1, patches.shape[1])
    rows = torch.randperm(flat.shape[0], generator=torch.Generator().manual_seed(4))[:512]
    fixed = torch.full((1, flat.shape[1]), scale, dtype=torch.float32)
    q, xs = oracle.input_tiles(flat[rows], CONFIG4, fixed)
    packed, ws = oracle.weight_tiles(source.weight.detach().cpu().flatten(1), CONFIG4)
    seed = oracle.name_seed(CONFIG4.seed, matrix.name)
    assert hip.mm_kernel(CONFIG4, flat.shape[0], q.shape[1], packed.shape[1]) == 2
    totals = gpu_totals(q.to(hip_device), packed.to(hip_device), CONFIG4, seed, 0)
    got_rows = got.flatten(2).transpose(1, 2).reshape(-1, source.out_channels)[rows.to(hip_device)]
    check_read(CONFIG4, got_rows, q, xs, packed, ws, seed, 0, totals, label=f"config4 {name}")


def test_config4_resnet18_batch_permutation(hip_device):
    """BASELINE config 4 at full size (batch 64, 224^2, every Conv2d/Linear converted,
    fixed input scales from a 4-batch synthetic calibration): with element-wise input
    quantization and cell-keyed noise, permuting the batch permutes the logits bit for
    bit."""
    torch.manual_seed(135)
    model = resnet18().to(hip_device)
    maxima = {}
    hooks = [module.register_forward_pre_hook(
        lambda module, inputs, name=name: maxima.__setitem__(
            name, max(maxima.get(name, 0.0), float(inputs[0].detach().abs().amax()))))
        for name, module in model.named_modules() if isinstance(module, (nn.Conv2d, nn.Linear))]
    with torch.no_grad():
        for _ in range(4):
            model(torch.randn(8, 3, 224, 224, device=hip_device))
    for hook in hooks:
        hook.remove()
    analog = convert_model(model, Simulator(CONFIG4, device=hip_device))
    for name, module in analog.named_modules():
        if name in maxima:
            matrices = module.matrices if hasattr(module, "matrices") else [module]
            for matrix in matrices:
                matrix.set_input_scale(max(maxima[name], 1.1754943508222875e-38) / 127)
    images = torch.randn(64, 3, 224, 224, device=hip_device)
    perm = torch.randperm(64, generator=torch.Generator().manual_seed(5)).to(hip_device)
    with torch.no_grad():
        logits = analog(images)
        reset_read_events(analog)
        permuted = analog(images[perm])
    assert logits.shape == (64, 1000) and torch.isfinite(logits).all()
    assert bits_equal(permuted, logits[perm])


# ---------------------------------------------------------------------------
# Config 5: LLM decoder linear shapes, BFP16 inputs (bw_e 8) x INT4 weights, drift + read noise
# ---------------------------------------------------------------------------
CONFIG5 = dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
               weight_slice=(1, 1, 2), bw_e=8, adc_bits=(6, 6, 7))
CONFIG5_NOISE = Nonidealities(read_variation=0.01, drift_coefficient=0.05, drift_time=100.0)


def _config5_tokens(tokens, features, seed):
    """Activations randn with 1% outlier channels x20."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, features, generator=gen)
    x[:, torch.randperm(features, generator=gen)[:features // 100]] *= 20
    return x


@pytest.mark.parametrize("mode", ["default", "tuned"])
def test_config5_up_proj_full_size_row_permutation(hip_device, tmp_path, mode):
    """The up/gate projection at full size (2048 tokens, 4096 -> 11008) on the wide MFMA
    read.  Input groups are per row (input_quant_gran (1, None)) and the read noise is keyed
    by cell and read event, so permuting the tokens permutes the output rows bit for bit:
    every row is computed at its new position with the same codes, scales and noise."""
    cfg = Config(**CONFIG5, nonidealities=CONFIG5_NOISE)
    x = _config5_tokens(2048, 4096, 55)
    gen = torch.Generator().manual_seed(56)
    w = torch.randn(4096, 11008, generator=gen) * 0.02
    rows, cols = cfg.array_size
    assert hip.mm_kernel(cfg, 2048, 4096 // rows, 11008 // cols) == 3
    perm = torch.randperm(2048, generator=gen)
    x_dev, w_dev = x.to(hip_device), w.to(hip_device)
    kwargs = dict(mode="tuned", cache_dir=tmp_path) if mode == "tuned" else {}
    say("config5 up_proj 2048x4096 @ 4096x11008", mode)
    out = Simulator(cfg, device=hip_device, **kwargs).mm(x_dev, w_dev)
    permuted = Simulator(cfg, device=hip_device, **kwargs).mm(x_dev[perm.to(hip_device)], w_dev)
    torch.cuda.synchronize()
    assert out.shape == (2048, 11008) and bool(torch.isfinite(out).all())
    assert bits_equal(permuted, out[perm.to(hip_device)])
    assert not bits_equal(permuted, out)


def test_config5_down_proj_rows_against_oracle(hip_device):
    """The down projection (11008 -> 4096) at full K: sampled rows of the GPU product against
    the oracle's read of the same rows (its own conductance samples), flip-aware, in the
    first and last two-tile chunks of columns."""
    cfg = Config(**CONFIG5, nonidealities=CONFIG5_NOISE)
    x = _config5_tokens(64, 11008, 57)
    gen = torch.Generator().manual_seed(58)
    w = torch.randn(11008, 4096, generator=gen) * 0.02
    out = Simulator(cfg, device=hip_device).mm(x.to(hip_device), w.to(hip_device))
    rows = torch.tensor([0, 17, 63])
    q, xs = oracle.input_tiles(x[rows], cfg)
    packed, ws = oracle.weight_tiles(w.T, cfg)
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, 0)
    got = out[rows.to(hip_device)].cpu()
    c = cfg.array_size[1]
    p = packed.shape[1]
    for first in (0, p - 2):
        tiles = (first, first + 2)
        check_read(cfg, got[:, first * c:(first + 2) * c], q, xs, packed, ws, seed, 0, totals,
                   tiles=tiles, label=f"config5 down_proj rows, tiles {tiles}")
