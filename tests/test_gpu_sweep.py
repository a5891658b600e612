"""Seeded sweep over configurations: Simulator.mm on the GPU against the oracle.

Each case draws a valid Config (bit widths, slicings, BFP exponents, signed or unsigned
weights, array shapes, rows per read, quantization groups, ADC widths and, for the noisy
half, device effects) and operand shapes that are not multiples of the arrays (up to 150
vectors), then checks the product as the
other parity tests do: bit for bit with ideal devices, flip-aware with device noise
(``tests/parity.py``).  The draws cover every read kernel (``hip.mm_kernel``); the CPU
test checks that the generator reaches them all without a GPU.
"""

import numpy as np
import pytest
import torch

from memfast_amd import Config, Nonidealities, hip
from parity import check_product, say

CASES = 24


def _slices(rng, bits, signed=True):
    """None (binary slices) or MSB-first widths summing to ``bits`` (a one-bit sign slice
    first when signed)."""
    if rng.random() < 0.2:
        return None
    widths = [1] if signed else []
    left = bits - sum(widths)
    while left > 0:
        width = int(min(left, rng.integers(1, 5)))
        widths.append(width)
        left -= width
    return tuple(widths)


def _config(rng, noisy):
    """A valid Config drawn from ``rng`` (redrawn until the constructor accepts it)."""
    while True:
        rows = int(rng.choice([32, 64, 128]))
        cols = int(rng.choice([16, 32, 64]))
        read_rows = int(rng.choice([d for d in (16, 32, 64, rows) if d <= rows and rows % d == 0]))
        wide = rng.random() < 0.2
        abits = int(rng.choice([12, 16])) if wide else int(rng.choice([4, 6, 8]))
        wbits = int(rng.choice([4, 6, 8]))
        bw_e = int(rng.integers(3, 9)) if wide and rng.random() < 0.5 else None
        signed = bw_e is not None or rng.random() < 0.85
        wslice = _slices(rng, wbits, signed)
        n_w = len(wslice) if wslice is not None else wbits
        adc = (tuple(int(rng.integers(4, 10)) for _ in range(n_w)) if rng.random() < 0.5
               else int(rng.integers(4, 10)))
        wgran = [(None, 1), (read_rows, 1), (None, None), (rows, 1)][int(rng.integers(4))]
        igran = [(1, None), (1, read_rows), (None, None), (1, rows)][int(rng.integers(4))]
        effects = dict(write_variation=0.0)
        if noisy:
            effects = dict(write_variation=float(rng.choice([0.01, 0.03])))
            kind = int(rng.integers(6))
            if kind == 1:
                effects.update(read_variation=0.01, adc_nonlinearity=0.1)
            elif kind == 2:
                effects.update(read_variation=0.02, read_mode="slice_pair")
            elif kind == 3:
                effects.update(read_variation=0.02, read_mode="output")
                # Half of them with voltage variation too, chosen from values already drawn
                # so that every other draw stays as it was.
                if (rows // 32 + cols // 16 + read_rows // 16) % 2:
                    effects.update(voltage_variation=0.02)
            elif kind == 4:
                effects.update(voltage_variation=0.02)
            elif kind == 5:
                effects.update(stuck_at_low=0.02, stuck_at_high=0.01, drift_coefficient=0.05,
                               drift_time=100.0)
        try:
            return Config(activation_bits=abits, weight_bits=wbits,
                          input_slice=_slices(rng, abits), weight_slice=wslice, bw_e=bw_e,
                          array_size=(rows, cols), rows_per_read=read_rows,
                          weight_quant_gran=wgran, input_quant_gran=igran, adc_bits=adc,
                          seed=int(rng.integers(0, 2**32)), weight_signed=signed,
                          nonidealities=Nonidealities(**effects))
        except ValueError:
            continue


def _case(index, noisy):
    rng = np.random.default_rng(1000 * int(noisy) + index)
    cfg = _config(rng, noisy)
    rows, cols = cfg.array_size
    n = int(rng.integers(1, 25)) if rng.random() < 0.7 else int(rng.integers(25, 150))
    k = int(rng.integers(1, 3 * rows + 1))
    o = int(rng.integers(1, 2 * cols + 6))
    gen = torch.Generator().manual_seed(index)
    a = torch.randn(n, k, generator=gen)
    b = torch.randn(k, o, generator=gen)
    if rng.random() < 0.25:
        a = a.relu()
    if not cfg.weight_signed:
        b = b.abs()   # unsigned weights are nonnegative INT values
    return cfg, a, b


def _kernel(cfg, n, k, o):
    rows, cols = cfg.array_size
    return hip.mm_kernel(cfg, n, -(-k // rows), -(-o // cols))


def test_sweep_reaches_every_read_kernel():
    """The draws cover the general kernel and both MFMA reads with noise, and the ideal
    MFMA read (at the shapes the product runs them)."""
    kinds = set()
    for noisy in (False, True):
        for index in range(CASES):
            cfg, a, b = _case(index, noisy)
            kinds.add(_kernel(cfg, a.shape[0], a.shape[1], b.shape[1]))
    assert {0, 1, 2, 3} <= kinds, kinds


@pytest.mark.gpu
@pytest.mark.parametrize("noisy", [False, True], ids=["ideal", "noisy"])
@pytest.mark.parametrize("index", range(CASES))
def test_sweep_product_matches_oracle(hip_device, index, noisy):
    from memfast_amd import Simulator

    cfg, a, b = _case(index, noisy)
    say("sweep", "noisy" if noisy else "ideal", index, tuple(a.shape), tuple(b.shape),
        "kernel", _kernel(cfg, a.shape[0], a.shape[1], b.shape[1]), cfg)
    sim = Simulator(cfg, device=hip_device)
    got = sim.mm(a.to(hip_device), b.to(hip_device))
    check_product(cfg, got, a, b, hip_device, label=f"sweep {index}")


FUSED_CASES = 12


def _fused_case(index):
    """A configuration and shapes that the two-launch route (hip.mm_from_float) takes: ideal
    devices, 32 rows per read, groups of one read on both sides, whole arrays; slicings,
    widths and ADC bits drawn.  Three operand pairs whose magnitudes range over 10^-12 to
    10^12, and sometimes A's far above the bound under which no FP32 restore can overflow
    (with B small enough that the product stays finite)."""
    rng = np.random.default_rng(7000 + index)
    while True:
        rows, cols = int(rng.choice([128, 256])), int(rng.choice([64, 128]))
        abits, wbits = int(rng.choice([4, 6, 8])), int(rng.choice([4, 6, 8]))
        wslice = _slices(rng, wbits)
        n_w = len(wslice) if wslice is not None else wbits
        adc = (tuple(int(rng.integers(4, 10)) for _ in range(n_w)) if rng.random() < 0.5
               else int(rng.integers(4, 10)))
        try:
            cfg = Config(activation_bits=abits, weight_bits=wbits, input_slice=_slices(rng, abits),
                         weight_slice=wslice, array_size=(rows, cols), rows_per_read=32,
                         weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=adc,
                         seed=int(rng.integers(0, 2**32)),
                         nonidealities=Nonidealities(write_variation=0.0))
        except ValueError:
            continue
        n = int(rng.integers(1, 200))
        k, o = rows * int(rng.integers(1, 5)), cols * int(rng.integers(1, 5))
        if hip.from_float_applies(cfg, n, k, o):
            break
    gen = torch.Generator().manual_seed(7000 + index)
    pairs = []
    for _ in range(3):
        a, b = torch.randn(n, k, generator=gen), torch.randn(k, o, generator=gen)
        if rng.random() < 0.3:
            a, b = a * 1e18, b * 1e-12
        else:
            a, b = a * 10.0 ** rng.uniform(-12, 12), b * 10.0 ** rng.uniform(-12, 12)
        pairs.append((a, b))
    return cfg, pairs


@pytest.mark.gpu
@pytest.mark.parametrize("index", range(FUSED_CASES))
def test_sweep_fused_products_back_to_back(hip_device, index):
    """Three products of one shape on one simulator with no synchronization between them:
    each call returns once its quantizers' status is published (or, above the overflow
    bound, after its read), and each output equals the oracle's bit for bit."""
    from memfast_amd import Simulator

    cfg, pairs = _fused_case(index)
    a0, b0 = pairs[0]
    say("fused sweep", index, tuple(a0.shape), tuple(b0.shape), cfg)
    sim = Simulator(cfg, device=hip_device)
    outs = [sim.mm(a.to(hip_device), b.to(hip_device)) for a, b in pairs]
    for call, ((a, b), got) in enumerate(zip(pairs, outs)):
        check_product(cfg, got, a, b, hip_device, label=f"fused {index}.{call}")


CONV_CASES = 8


def _conv(index, noisy):
    """A drawn configuration with a Conv2d geometry (kernel, stride, padding, dilation,
    groups) and its input."""
    rng = np.random.default_rng(5000 + 1000 * int(noisy) + index)
    cfg = _config(rng, noisy)
    groups = int(rng.choice([1, 1, 2]))
    channels = groups * int(rng.integers(1, 5))
    out_channels = groups * int(rng.integers(1, 4))
    kernel = (int(rng.integers(1, 5)), int(rng.integers(1, 5)))
    stride = (int(rng.integers(1, 3)), int(rng.integers(1, 3)))
    padding = (int(rng.integers(0, 3)), int(rng.integers(0, 3)))
    dilation = (int(rng.integers(1, 3)), int(rng.integers(1, 3)))
    size = (int(rng.integers(8, 14)), int(rng.integers(8, 14)))
    torch.manual_seed(index)
    source = torch.nn.Conv2d(channels, out_channels, kernel, stride, padding, dilation, groups)
    if not cfg.weight_signed:
        with torch.no_grad():
            source.weight.abs_()
    x = torch.randn(int(rng.integers(1, 4)), channels, *size)
    return cfg, source, x


@pytest.mark.gpu
@pytest.mark.parametrize("noisy", [False, True], ids=["ideal", "noisy"])
@pytest.mark.parametrize("index", range(CONV_CASES))
def test_sweep_conv2d_matches_oracle(hip_device, index, noisy):
    """AnalogConv2d (implicit im2col where it applies) against the oracle's read of
    F.unfold's patch matrix, group by group."""
    from torch.nn import functional as F

    from memfast_amd import Simulator
    from memfast_amd.nn import AnalogConv2d

    cfg, source, x = _conv(index, noisy)
    say("conv sweep", "noisy" if noisy else "ideal", index, source, tuple(x.shape), cfg)
    layer = AnalogConv2d(source.to(hip_device), Simulator(cfg, device=hip_device), name="conv")
    got = layer(x.to(hip_device))
    source = source.cpu()
    patches = F.unfold(x, source.kernel_size, source.dilation, source.padding, source.stride)
    groups, out_channels = source.groups, source.out_channels
    size = source.in_channels // groups * source.kernel_size[0] * source.kernel_size[1]
    per_group = out_channels // groups
    rows = got.flatten(2).transpose(1, 2)            # [N, L, out_channels]
    for g in range(groups):
        block = slice(g * per_group, (g + 1) * per_group)
        check_product(cfg, rows[:, :, block],
                      patches[:, g * size:(g + 1) * size].transpose(1, 2),
                      source.weight[block].flatten(1).T, hip_device, name=f"conv.group{g}",
                      bias=source.bias[block], label=f"conv sweep {index} group {g}")


FIXED_CASES = 16


def _fixed(index):
    """A drawn configuration, inputs and a fixed per-feature input scale; a quarter of the
    inputs sit on or next to half-integer quotients of their scale."""
    rng = np.random.default_rng(9000 + index)
    cfg = _config(rng, False)
    n, k = int(rng.integers(1, 40)), int(rng.integers(1, 3 * cfg.array_size[0] + 1))
    scale = torch.from_numpy(np.exp(rng.uniform(-6.0, 2.0, (1, k))).astype(np.float32))
    gen = torch.Generator().manual_seed(index)
    x = torch.randn(n, k, generator=gen) * 4.0
    limit = 1 << (cfg.activation_bits - 1)
    ties = torch.from_numpy(rng.integers(-limit - 1, limit + 1, (n, k)).astype(np.float64) + 0.5)
    near = (ties * scale.double()).float()
    pick = torch.from_numpy(rng.random((n, k)) < 0.25)
    x = torch.where(pick, near, x)
    return cfg, x, scale


@pytest.mark.gpu
@pytest.mark.parametrize("index", range(FIXED_CASES))
def test_sweep_fixed_scale_input_tiles(hip_device, index):
    """Input codes and per-read scales with a fixed (calibrated) per-feature scale, narrow
    and wide configurations, bit for bit against the oracle (codes past the range clamp)."""
    from oracle import oracle

    cfg, x, scale = _fixed(index)
    say("fixed-scale sweep", index, tuple(x.shape), cfg)
    q, xs = hip.input_tiles(x.to(hip_device), cfg, scale.to(hip_device))
    q_ref, xs_ref = oracle.input_tiles(x, cfg, scale)
    mask = (1 << cfg.activation_bits) - 1
    assert torch.equal(q.cpu().to(torch.int64) & mask, q_ref.to(torch.int64) & mask)
    assert torch.equal(xs.cpu(), xs_ref)


TUNED_CASES = 40


@pytest.mark.gpu
@pytest.mark.parametrize("noisy", [False, True], ids=["ideal", "noisy"])
@pytest.mark.parametrize("index", range(TUNED_CASES))
def test_sweep_tuned_product_matches_oracle(hip_device, tmp_path, index, noisy):
    """Tuned mode (its schedule search, cache write and selected kernel) gives the product
    default mode gives: the oracle's, as in test_sweep_product_matches_oracle."""
    from memfast_amd import Simulator

    cfg, a, b = _case(100 + index, noisy)
    say("tuned sweep", "noisy" if noisy else "ideal", index, tuple(a.shape), tuple(b.shape), cfg)
    sim = Simulator(cfg, mode="tuned", device=hip_device, cache_dir=tmp_path)
    got = sim.mm(a.to(hip_device), b.to(hip_device))
    check_product(cfg, got, a, b, hip_device, label=f"tuned sweep {index}")


GRU_CASES = 6


@pytest.mark.gpu
@pytest.mark.parametrize("noisy", [False, True], ids=["ideal", "noisy"])
@pytest.mark.parametrize("index", range(GRU_CASES))
def test_sweep_gru_sequence_matches_oracle_steps(hip_device, index, noisy):
    """AnalogGRU over a sequence (the native sequence call where it applies) against its
    steps recomputed from PyTorch's gate equations over oracle-checked reads."""
    from memfast_amd import Simulator
    from memfast_amd.nn import AnalogGRU
    from parity import gru_step_parity

    rng = np.random.default_rng(7000 + 1000 * int(noisy) + index)
    cfg = _config(rng, noisy)
    hidden = int(rng.choice([16, 48, 64]))
    inputs = int(rng.integers(4, 41))
    steps, batch = int(rng.integers(3, 6)), int(rng.integers(1, 5))
    torch.manual_seed(index)
    source = torch.nn.GRU(inputs, hidden, num_layers=1)
    if not cfg.weight_signed:
        with torch.no_grad():
            for weight in (source.weight_ih_l0, source.weight_hh_l0):
                weight.abs_()
    x = torch.randn(steps, batch, inputs)
    say("gru sweep", "noisy" if noisy else "ideal", index, source, tuple(x.shape), cfg)
    layer = AnalogGRU(source.to(hip_device), Simulator(cfg, device=hip_device), name="gru")
    output, _ = layer(x.to(hip_device))
    gru_step_parity(layer.cells[0], source.cpu(), x, output, hip_device, label=f"gru sweep {index}")


def _injected_flips(cfg, a, b, device, events, tolerance=2.0**-16):
    """Per read event, the kernel's slice totals (the one hip.mm runs) against oracle.partial,
    both given the oracle's own sampled conductances.  Every differing total must be explained
    by flips of pairs whose exact ADC argument (oracle.flips.adc_arguments) lies within
    ``tolerance`` (relative) of a rounding boundary.  Returns the flips per event, the codes
    per event and the largest relative boundary distance of a flipped pair."""
    from oracle import flips, oracle
    from parity import gpu_totals

    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    p = packed.shape[1]
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    q_dev, packed_dev = q.to(device), packed.to(device)
    counts, worst = [], 0.0
    for event in events:
        raw, _, _ = oracle.restored(packed, cfg, seed, event, 0, p)
        expected = oracle.partial(q, packed, cfg, seed, event, 0, p, conductance=raw)
        got = gpu_totals(q_dev, packed_dev, cfg, seed, event, conductance=raw.to(device))
        arguments = flips.adc_arguments(q, packed, cfg, raw)
        _, flipped, far, unexplained = flips.boundary_flips(cfg, got, expected, arguments,
                                                            tolerance)
        assert not unexplained, (event, unexplained[:3])
        counts.append(flipped)
        worst = max(worst, far)
    codes = expected.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    return counts, codes, worst


@pytest.mark.gpu
def test_sweep_draw_1386_injected_conductances(hip_device):
    """Regression for product draw 1386 with noise (9-bit S-curve ADCs, shared read noise,
    4-bit inputs, 12 x 54 @ 54 x 57 on 32 x 32 arrays), which once flipped 2 of its 13,824
    codes against the oracle's sampled conductances, more than 1e-4 of that one read.
    Given the oracle's own conductances, over 64 read events every flipped code is a
    rounding-boundary flip (its exact argument within 2^-16 relative of a half-integer)
    and the flips stay within 1e-4 of all codes."""
    cfg, a, b = _case(1386, True)
    assert cfg.nonidealities.adc_nonlinearity and max(cfg.adc_bits) >= 9
    assert _kernel(cfg, *a.shape, b.shape[1]) == 2
    counts, codes, worst = _injected_flips(cfg, a, b, hip_device, range(64))
    say("draw 1386 injected: flips per event", counts, "of", codes, "codes each; largest "
        "relative boundary distance of a flip", worst)
    assert sum(counts) <= 1e-4 * codes * len(counts)
