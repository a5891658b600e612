"""GPU parity of the gfx950 kernels against the CPU oracle and the reference's vectors.

Bar: bit-exact for codes, scales, packing, RNG uniforms and every ideal-device
output; with device noise, identical ADC codes given injected conductances
except rounding-boundary flips (<= 1e-4 of codes) and output relative error
<= 1e-5 elsewhere (the BASELINE tolerance).  Noisy products are checked with
``oracle.flips.check_noisy`` on the slice totals behind each output: flipped
codes at most 1e-4 of all codes, every output whose totals all match within
1e-5 relative, every other output within the effect of its own flips.
"""

import ctypes as ct
import math

import numpy as np
import pytest
import torch

from memfast_amd import Config, Nonidealities, hip
from oracle import flips, oracle
from parity import check_product, gpu_totals, oracle_totals

pytestmark = pytest.mark.gpu

CONFIG2 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
               weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
               weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))


def say(*args):
    print("[gpu-parity]", *args, flush=True)


class BitsEqual:
    """Truthy bitwise comparison whose repr explains a mismatch."""

    def __init__(self, a, b):
        a, b = a.detach().cpu().contiguous(), b.detach().cpu().contiguous().to(a.dtype)
        assert a.shape == b.shape, (a.shape, b.shape)
        if a.dtype.is_floating_point:
            view = torch.int32 if a.dtype == torch.float32 else torch.int64
            diff = a.view(view) != b.view(view)
        else:
            diff = a != b
        self.ok = not bool(diff.any())
        self.count = int(diff.sum())
        self.total = diff.numel()
        self.max_abs = float((a.double() - b.double()).abs().max()) if self.count else 0.0
        self.first = diff.nonzero()[:3].tolist() if self.count else []

    def __bool__(self):
        return self.ok

    def __repr__(self):
        return (f"BitsEqual({self.count}/{self.total} differ, max |diff| {self.max_abs:.3e}, "
                f"first at {self.first})")


def bits_equal(a, b):
    return BitsEqual(a, b)


def ideal(**kwargs):
    return Config(**kwargs, nonidealities=Nonidealities(write_variation=0.0))


IDEAL_CASES = [
    ("config1", ideal(**CONFIG2 | dict(adc_bits=7)), 4, 128, 32),
    ("config2_small", ideal(**CONFIG2), 70, 512, 300),
    ("binary8_64", ideal(input_slice=(1,) * 8, weight_slice=(1,) * 8, array_size=(64, 64),
                         adc_bits=8, input_quant_gran=(1, 64)), 9, 200, 130),
    ("int4_weights", ideal(weight_bits=4, array_size=(64, 64), adc_bits=6), 5, 150, 70),
    ("p64_256", ideal(**CONFIG2 | dict(array_size=(256, 256), rows_per_read=64, adc_bits=8,
                                       weight_quant_gran=(None, 1), input_quant_gran=(1, 64))),
     33, 300, 260),
    ("ragged_general", ideal(array_size=(20, 8), rows_per_read=7, adc_bits=4), 6, 45, 19),
    ("narrow_cols", ideal(array_size=(32, 12), rows_per_read=16, adc_bits=5,
                          weight_slice=(1, 3, 4)), 5, 70, 30),
    ("unsigned", ideal(weight_bits=4, weight_signed=False, weight_slice=(2, 2),
                       array_size=(32, 16), adc_bits=5), 4, 40, 20),
    # Quantization routes: 2-D groups (atomic group maxima) on both operands ...
    ("grouped_2d", ideal(array_size=(64, 32), rows_per_read=16, adc_bits=8,
                         input_quant_gran=(2, 16), weight_quant_gran=(32, 4)), 7, 150, 40),
    # ... scalar loads and byte stores (odd group width, 66-row tiles) ...
    ("odd_rows", ideal(array_size=(66, 32), adc_bits=8, input_quant_gran=(1, 66),
                       weight_quant_gran=(66, 1)), 5, 150, 36),
    # ... and groups too long for one thread (whole rows and whole columns),
    ("whole_rows", ideal(adc_bits=8), 3, 1500, 20),
    # one wave per 1024-float row group,
    ("row_wave", ideal(adc_bits=8), 3, 1024, 20),
    # LDS-tiled weight groups with a ragged last group and padded columns,
    ("tile_ragged", ideal(array_size=(64, 64), rows_per_read=16, weight_quant_gran=(16, 1),
                          input_quant_gran=(1, 16), adc_bits=8), 5, 150, 100),
    # register column groups with byte stores (kp = 54 is not a multiple of 4).
    ("col_bytes", ideal(array_size=(18, 32), rows_per_read=2, weight_quant_gran=(8, 1),
                        adc_bits=6), 4, 45, 36),
]


@pytest.mark.parametrize("name,cfg,n,k,o", IDEAL_CASES, ids=[c[0] for c in IDEAL_CASES])
def test_tiles_bit_exact(hip_device, name, cfg, n, k, o):
    say("tiles", name, n, k, o)
    gen = torch.Generator().manual_seed(11)
    a = torch.randn(n, k, generator=gen)
    b = torch.randn(k, o, generator=gen)
    if not cfg.weight_signed:
        b = b.abs()
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, packed_t, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    torch.cuda.synchronize()
    assert bits_equal(q, q_ref) and bits_equal(xs, xs_ref)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)
    m, p, r, c = packed_ref.shape
    expected_t = packed_ref.permute(1, 3, 0, 2).reshape(p * c, m * r)
    assert bits_equal(packed_t, expected_t)
    assert bits_equal(hip.transpose_packed(packed, cfg), expected_t)


def test_fixed_input_scale(hip_device):
    cfg = ideal(array_size=(32, 16), rows_per_read=16)
    a = torch.randn(7, 50) * 3
    scale = torch.full((1, 50), 0.0123)
    q, xs = hip.input_tiles(a.to(hip_device), cfg, scale.to(hip_device))
    q_ref, xs_ref = oracle.input_tiles(a, cfg, scale)
    assert bits_equal(q, q_ref) and bits_equal(xs, xs_ref)


@pytest.mark.parametrize("name,cfg,n,k,o", IDEAL_CASES, ids=[c[0] for c in IDEAL_CASES])
def test_ideal_mm_bit_exact(hip_device, name, cfg, n, k, o):
    say("ideal mm", name, n, k, o)
    gen = torch.Generator().manual_seed(5)
    a = torch.randn(n, k, generator=gen)
    b = torch.randn(k, o, generator=gen)
    if not cfg.weight_signed:
        b = b.abs()
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    expected = oracle.execute(q_ref, xs_ref, packed_ref, ws_ref, cfg, seed, 0, o)
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, packed_t, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    p, c = packed.shape[1], cfg.array_size[1]
    kernel = hip.mm_kernel(cfg, n, q.shape[1], p)
    say("  kernel", kernel)
    out = hip.mm(q, xs, packed, packed_t, ws.reshape(-1, p * c), cfg, seed, 0)
    assert bits_equal(out[:, :o], expected)
    # The general kernel agrees bit for bit as well.
    general = hip.mm(q, xs, packed, None, ws.reshape(-1, p * c), cfg, seed, 0)
    assert bits_equal(general[:, :o], expected)


def test_mfma_kernel_selected_for_baseline(hip_device):
    cfg = ideal(**CONFIG2)
    assert hip.mm_kernel(cfg, 4096, 32, 32) == 1
    noisy = Config(**CONFIG2)   # default write variation
    assert hip.mm_kernel(noisy, 4096, 32, 32) == 2
    for mode in ("slice_pair", "output"):
        other = Config(**CONFIG2, nonidealities=Nonidealities(read_variation=0.01, read_mode=mode))
        assert hip.mm_kernel(other, 4096, 32, 32) == 2
    voltage = Config(**CONFIG2, nonidealities=Nonidealities(voltage_variation=0.01))
    assert hip.mm_kernel(voltage, 4096, 32, 32) == 2


@pytest.mark.parametrize("name,cfg,n,k,o", IDEAL_CASES[:4], ids=[c[0] for c in IDEAL_CASES[:4]])
def test_ideal_partial_totals(hip_device, name, cfg, n, k, o):
    say("partial", name)
    a = torch.randn(n, k)
    b = torch.randn(k, o)
    q_ref, _ = oracle.input_tiles(a, cfg)
    packed_ref, _ = oracle.weight_tiles(b.T, cfg)
    p = packed_ref.shape[1]
    begin, end = (1, p) if p > 1 else (0, 1)
    expected = oracle.partial(q_ref, packed_ref, cfg, 9, 0, begin, end)
    got = hip.partial(q_ref.to(hip_device), packed_ref.to(hip_device), cfg, None, 9, 0, begin, end)
    assert bits_equal(got, expected)


def test_dft_known_answer_gpu(hip_device):
    size = 256
    idx = np.arange(size)
    basis = np.exp(-2j * np.pi * np.outer(idx, idx) / size) / np.sqrt(size)
    weight = torch.tensor(basis.real, dtype=torch.float32)
    vectors = torch.linspace(-1, 1, 3 * size).reshape(3, size)
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1,) * 8, weight_slice=(1,) * 8,
                 array_size=(64, 64), adc_bits=8, input_quant_gran=(1, 64),
                 weight_quant_gran=(None, 1), seed=135,
                 nonidealities=Nonidealities(write_variation=0.0))
    from memfast_amd import Simulator

    sim = Simulator(cfg, device=hip_device)
    actual = sim.mm(vectors.to(hip_device), weight.to(hip_device)).cpu()
    assert bits_equal(actual, oracle.mm(vectors, weight, cfg))
    wscale = weight.abs().amax(dim=0, keepdim=True) / 127
    groups = vectors.reshape(3, size // 64, 64)
    iscale = (groups.abs().amax(dim=-1, keepdim=True) / 127).expand_as(groups).reshape_as(vectors)
    expected = ((vectors / iscale).round().clamp(-127, 127) * iscale) @ (
        (weight / wscale).round().clamp(-127, 127) * wscale)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=2e-5)


# ---------------------------------------------------------------------------
# RNG
# ---------------------------------------------------------------------------
def test_rng_uniform_bit_exact(hip_device, reference_vectors):
    v = reference_vectors
    addresses = torch.from_numpy(v["rng_address"]).to(hip_device)
    for si, seed in enumerate(v["rng_seeds"].tolist()):
        for ti, stream in enumerate(v["rng_streams"].tolist()):
            u = hip.rng(addresses, int(seed), int(stream), "uniform").cpu().numpy()
            np.testing.assert_array_equal(u, v["rng_uniform"][si, ti])
            z = hip.rng(addresses, int(seed), int(stream), "normal").cpu().numpy()
            np.testing.assert_allclose(z, v["rng_normal"][si, ti], rtol=2e-6, atol=2e-6)


# ---------------------------------------------------------------------------
# Noisy devices
# ---------------------------------------------------------------------------
NOISE = {
    "write": dict(write_variation=0.02),
    "shared": dict(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1),
    "slice_pair": dict(write_variation=0.02, read_variation=0.02, read_mode="slice_pair"),
    "output": dict(write_variation=0.02, read_variation=0.02, read_mode="output"),
    "voltage": dict(write_variation=0.0, voltage_variation=0.05),
    "saf_drift": dict(write_variation=0.02, stuck_at_low=0.05, stuck_at_high=0.03,
                      drift_coefficient=0.05, drift_time=100.0),
}
SMALL = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
             weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
             weight_quant_gran=(16, 1), input_quant_gran=(1, 16), adc_bits=(6, 7, 7, 8, 8))


@pytest.mark.parametrize("mode", list(NOISE))
def test_restore_close_to_oracle(hip_device, mode):
    cfg = Config(**SMALL, nonidealities=Nonidealities(**NOISE[mode]))
    b = torch.randn(70, 40)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    p = packed.shape[1]
    expected, _, _ = oracle.restored(packed, cfg, 1234, 3, 0, p)
    got = hip.restore(packed.to(hip_device), cfg, 1234, 3, 0, p).cpu()
    if got.shape[0] > 1:  # slice_pair planes: compare plane 0 to the oracle's factor applied
        got = got[0]
        cell = oracle.cell_addresses(*packed.shape[:2], len(cfg.weight_layout),
                                     *packed.shape[2:], 0, p)
        expected = expected * torch.exp(cfg.nonidealities.read_variation * oracle.normal(
            cell * len(cfg.input_layout), oracle.event_seed(1234, 3), 20))
    else:
        got = got[0]
    torch.testing.assert_close(got, expected, rtol=2e-6, atol=0)


@pytest.mark.parametrize("mode", list(NOISE))
def test_noisy_codes_with_injected_conductances(hip_device, mode):
    """Identical ADC codes except rounding-boundary flips (<= 1e-4)."""
    say("noisy codes", mode)
    cfg = Config(**SMALL, nonidealities=Nonidealities(**NOISE[mode]))
    gen = torch.Generator().manual_seed(21)
    a = torch.randn(24, 96, generator=gen)
    b = torch.randn(96, 48, generator=gen)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    p = packed.shape[1]
    seed, event = 777, 5
    raw, cell, read_seed = oracle.restored(packed, cfg, seed, event, 0, p)
    codes_ref = {}
    oracle.partial(q, packed, cfg, seed, event, 0, p, conductance=raw, codes=codes_ref)
    planes = hip.restore_planes(cfg)
    if planes > 1:
        a_count = len(cfg.input_layout)
        stack = [raw * torch.exp(cfg.nonidealities.read_variation * oracle.normal(
            cell * a_count + ai, read_seed, 20)) for ai in range(a_count)]
        injected = torch.stack(stack)
        # The oracle applies the slice-pair factor itself; give it the programmed raw.
    else:
        injected = raw[None]
    _, codes = hip.partial(q.to(hip_device), packed.to(hip_device), cfg, None, seed, event, 0, p,
                           conductance=injected.to(hip_device), codes=True)
    codes = codes.cpu()
    n, groups = q.shape[0], codes.shape[1]
    flips = 0
    total = 0
    for (ai, wi), ref in codes_ref.items():
        ref = ref.reshape(n, groups, p * cfg.array_size[1])
        got = codes[:, :, ai, wi, :]
        flips += (got != ref).sum().item()
        assert (got - ref).abs().max().item() <= 1
        total += ref.numel()
    say("  flips", flips, "of", total)
    assert flips <= max(1, 1e-4 * total)


@pytest.mark.parametrize("mode", list(NOISE))
def test_noisy_mm_matches_reference_vectors(hip_device, reference_vectors, mode):
    """Full Simulator.mm on the GPU against the reference CPU outputs (same seeds/events)."""
    from memfast_amd import Simulator

    v = reference_vectors
    cfg = Config(**SMALL, nonidealities=Nonidealities(**NOISE[mode]))
    a = torch.from_numpy(v[f"case_{mode}_a"]).to(hip_device)
    b = torch.from_numpy(v[f"case_{mode}_b"]).to(hip_device)
    sim = Simulator(cfg, device=hip_device)
    q = torch.from_numpy(v[f"case_{mode}_q"])
    packed = torch.from_numpy(v[f"case_{mode}_packed"])
    xs = torch.from_numpy(v[f"case_{mode}_xscale"])
    ws = torch.from_numpy(v[f"case_{mode}_wscale"])
    seed = int(v[f"case_{mode}_seed"])
    for event in (0, 1):
        got = sim.mm(a, b)
        totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, event)
        if event == 0:
            # The reference's own slice totals and output (same seed and event).
            ref_totals = torch.from_numpy(v[f"case_{mode}_totals"])
            ref = torch.from_numpy(v[f"case_{mode}_out0"])
        else:
            ref_totals = oracle_totals(q, packed, cfg, seed, event)
            ref = oracle.execute(q, xs, packed, ws, cfg, seed, event, b.shape[1],
                                 totals=ref_totals)
        say("  event", event, flips.check_noisy(cfg, got, ref, totals, ref_totals, xscale=xs,
                                                wscale=ws, label=f"{mode} event {event}"))


def test_ideal_simulator_matches_reference_vectors(hip_device, reference_vectors):
    from memfast_amd import Simulator

    v = reference_vectors
    cfg = Config(**SMALL, nonidealities=Nonidealities(write_variation=0.0))
    sim = Simulator(cfg, device=hip_device)
    a = torch.from_numpy(v["case_ideal_a"]).to(hip_device)
    b = torch.from_numpy(v["case_ideal_b"]).to(hip_device)
    assert bits_equal(sim.mm(a, b), torch.from_numpy(v["case_ideal_out0"]))
    assert bits_equal(sim.mm(a, b), torch.from_numpy(v["case_ideal_out1"]))


def test_lenet_checkpoint_codes_on_gpu(hip_device):
    from pathlib import Path

    data = np.load(Path(__file__).with_name("golden") / "lenet_int4.npz", allow_pickle=False)
    cfg = Config(activation_bits=8, weight_bits=4, array_size=(64, 64), adc_bits=6)
    for index in range(int(data["count"])):
        weight = torch.from_numpy(data[f"l{index}_weight"]).to(hip_device)
        packed, _, _ = hip.weight_tiles(weight, cfg)
        np.testing.assert_array_equal(packed.cpu().numpy(), data[f"l{index}_packed"])


def test_config2_full_size_rows(hip_device):
    """BASELINE config 2 (4096^3, ideal): GPU rows equal the oracle on a row sample.

    Input groups are per row (1,32), so any row subset quantizes identically.
    """
    cfg = ideal(**CONFIG2)
    torch.manual_seed(135)
    a = torch.randn(4096, 4096)
    b = torch.randn(4096, 4096)
    from memfast_amd import Simulator

    sim = Simulator(cfg, device=hip_device)
    say("config2 4096^3 ideal on GPU")
    out = sim.mm(a.to(hip_device), b.to(hip_device))
    rows = torch.tensor([0, 1, 777, 2048, 4095])
    say("oracle on rows", rows.tolist())
    expected = oracle.mm(a[rows], b, cfg)
    assert bits_equal(out[rows.to(hip_device)], expected)


def test_config2_full_size_permutation_equivariance(hip_device):
    """BASELINE config 2 at full size, every row and column: with per-row input groups (1, 32)
    and per-column weight groups (32, 1) an output element depends only on its row of A and
    its column of B, so permuting A's rows and B's columns permutes the output, bit for bit."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(136)
    a = torch.randn(4096, 4096, generator=gen)
    b = torch.randn(4096, 4096, generator=gen)
    rows = torch.randperm(4096, generator=gen)
    cols = torch.randperm(4096, generator=gen)
    say("config2 4096^3 permutation equivariance")
    out = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    permuted = Simulator(cfg, device=hip_device).mm(a[rows].to(hip_device),
                                                    b[:, cols].contiguous().to(hip_device))
    expected = out.cpu()[rows][:, cols]
    assert bits_equal(permuted, expected)
    assert not torch.equal(permuted.cpu(), out.cpu())   # the permutation moved values


FROM_FLOAT_SHAPES = [(1, 128, 128), (37, 256, 128), (64, 128, 256), (200, 384, 256),
                     (130, 4096, 128)]


@pytest.mark.parametrize("data", ["randn", "saturating"])
@pytest.mark.parametrize("n,k,o", FROM_FLOAT_SHAPES)
def test_mm_from_float_matches_separate_calls(hip_device, n, k, o, data):
    """mf_mm_from_float (one launch quantizing both operands and reducing the digit masks,
    then the read) writes exactly what mf_quantize_inputs, mf_quantize_weights and mf_mm
    write: codes, scale tables, the digit masks in the workspace and the output, which is
    the oracle's.  Saturating operands make every clamp candidate real."""
    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(n * 7 + k + o)
    a, b = torch.randn(n, k, generator=gen), torch.randn(k, o, generator=gen)
    if data == "saturating":
        a, b = a.sign(), b.sign()
    ad, bd = a.to(hip_device), b.to(hip_device)
    assert hip.from_float_applies(cfg, n, k, o)
    m, p = k // 128, o // 128
    ws1 = torch.zeros(hip.mm_workspace_bytes(cfg, n, m, p), dtype=torch.uint8, device=hip_device)
    ws2 = torch.zeros_like(ws1)
    s1, s2 = hip.status_word(hip_device), hip.status_word(hip_device)
    q, xscale, (packed, packed_t, wscale), out = hip.mm_from_float(ad, bd, cfg, status=s1,
                                                                   workspace=ws1)
    packed2, packed_t2, wscale2 = hip.weight_tiles(bd.T, cfg, status=s2)
    q2, xscale2 = hip.input_tiles(ad, cfg, status=s2)
    out2 = hip.mm(q2, xscale2, packed2, packed_t2, wscale2.reshape(-1, o), cfg, 0, 0,
                  status=s2, workspace=ws2, out_cols=o, k_rows=k)
    for name, got, want in (("q", q, q2), ("xscale", xscale, xscale2), ("packed", packed, packed2),
                            ("packed_t", packed_t, packed_t2), ("wscale", wscale, wscale2),
                            ("out", out, out2)):
        assert bits_equal(got, want), name
    G = m * cfg.reads_per_array
    xwords, wwords = -(-n // 64) * G, (o // 32) * G
    xbytes = -(-xwords * 8 // 256) * 256
    for lo, count in ((0, xwords), (xbytes, wwords)):
        got = ws1[lo:lo + 8 * count].view(torch.int64)
        want = ws2[lo:lo + 8 * count].view(torch.int64)
        assert torch.equal(got, want), (lo, count)
    assert int(s1.item()) == int(s2.item()) == 0
    assert bits_equal(out, oracle.mm(a, b, cfg))


def near_half_integer_groups(count, seed):
    """[count, 32] float32 groups whose quotients x / s (s = peak / 127, as the quantizer
    computes it) sit on or within three ulps of a half-integer: exact ties (power-of-two
    scales), their neighbours, and groups with subnormal and huge peaks."""
    rng = np.random.default_rng(seed)
    groups = np.empty((count, 32), dtype=np.float32)
    for g in range(count):
        kind = g % 4
        if kind == 0:
            peak = np.float32(127.0 * 2.0 ** rng.integers(-20, 20))   # s a power of two
        elif kind == 1:
            peak = np.float32(np.exp(rng.uniform(-8.0, 8.0)))
        elif kind == 2:
            peak = np.float32(rng.uniform(1e-43, 1e-39))              # subnormal scale
        else:
            peak = np.float32(rng.uniform(1e30, 3e38))
        s = max(np.float32(peak) / np.float32(127.0), np.float32(1e-45))
        groups[g, 0] = peak if rng.integers(2) else -peak
        for r in range(1, 32):
            x = np.float32((rng.integers(-127, 127) + 0.5) * np.float64(s))
            for _ in range(abs(step := int(rng.integers(-3, 4)))):
                x = np.nextafter(x, np.float32(np.inf if step > 0 else -np.inf), dtype=np.float32)
            groups[g, r] = np.clip(x, -peak, peak)
    return torch.from_numpy(groups)


def test_mm_from_float_codes_at_half_integer_quotients(hip_device):
    """The fused quantizers divide by multiplying with the group's reciprocal and fall back to
    the division near half-integer quotients: codes and scales equal the oracle's (torch's
    true division) on operands built from ties and their ulp neighbours."""
    cfg = ideal(**CONFIG2)
    n, k, o = 64, 512, 128
    a = near_half_integer_groups(n * k // 32, 5).reshape(n, k)
    b = near_half_integer_groups(k * o // 32, 6).reshape(o, k // 32, 32).permute(1, 2, 0)
    b = b.reshape(k, o).contiguous()          # column groups of 32 rows
    assert hip.from_float_applies(cfg, n, k, o)
    q, xscale, (packed, _, wscale), _ = hip.mm_from_float(a.to(hip_device), b.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    assert bits_equal(q, q_ref)
    assert bits_equal(xscale.reshape(xs_ref.shape), xs_ref)
    assert bits_equal(packed, packed_ref)
    assert bits_equal(wscale.reshape(ws_ref.shape), ws_ref)


def test_mm_from_float_operand_forms(hip_device):
    """Simulator.mm on the two-launch route with half-precision operands, a transposed B
    (an nn.Linear weight read as W.T) and a sliced A: the oracle's result in A's dtype."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(10)
    a = torch.randn(96, 512, generator=gen)
    w = torch.randn(256, 512, generator=gen)          # [O, K]
    sim = Simulator(cfg, device=hip_device)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        ad, wd = a.to(hip_device, dtype), w.to(hip_device, dtype)
        assert hip.from_float_applies(cfg, 96, 512, 256)
        got = sim.mm(ad, wd.T)
        assert got.dtype == dtype
        assert bits_equal(got, oracle.mm(ad.cpu(), wd.T.cpu(), cfg))
    wide = torch.randn(96, 1024, generator=gen)
    got = sim.mm(wide.to(hip_device)[:, 256:768], w.to(hip_device).T)
    assert bits_equal(got, oracle.mm(wide[:, 256:768], w.T, cfg))


def test_mm_from_float_flags_nonfinite_operands(hip_device):
    """The fused quantizers set the status bits the separate ones set; Simulator.mm raises
    the reference's errors from them, A before B."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(9)
    a, b = torch.randn(64, 256, generator=gen), torch.randn(256, 128, generator=gen)
    bad_a, bad_b = a.clone(), b.clone()
    bad_a[5, 77] = float("nan")
    bad_b[200, 3] = float("-inf")
    for left, right, bit in ((bad_a, b, hip.STATUS_INPUT), (a, bad_b, hip.STATUS_WEIGHT),
                             (bad_a, bad_b, hip.STATUS_INPUT | hip.STATUS_WEIGHT)):
        status = hip.status_word(hip_device)
        assert hip.mm_from_float(left.to(hip_device), right.to(hip_device), cfg,
                                 status=status) is not None
        assert int(status.item()) & (hip.STATUS_INPUT | hip.STATUS_WEIGHT) == bit
    sim = Simulator(cfg, device=hip_device)
    with pytest.raises(ValueError, match="A must be finite"):
        sim.mm(bad_a.to(hip_device), bad_b.to(hip_device))
    with pytest.raises(ValueError, match="B must be finite"):
        sim.mm(a.to(hip_device), bad_b.to(hip_device))
    assert bits_equal(sim.mm(a.to(hip_device), b.to(hip_device)), oracle.mm(a, b, cfg))


def test_mm_from_float_publishes_status_when_the_read_starts(hip_device):
    """The read's first workgroup copies the quantizers' status bits to a pinned host word
    (hip.status_wait, mf_status_wait): the bits the device status word holds afterwards."""
    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(11)
    a, b = torch.randn(64, 256, generator=gen), torch.randn(256, 128, generator=gen)
    bad_a, bad_b = a.clone(), b.clone()
    bad_a[5, 77] = float("nan")
    bad_b[200, 3] = float("-inf")
    box = hip.mailbox()
    checks = hip.STATUS_INPUT | hip.STATUS_WEIGHT
    for left, right, bits in ((a, b, 0), (bad_a, b, hip.STATUS_INPUT),
                              (a, bad_b, hip.STATUS_WEIGHT)):
        status = hip.status_word(hip_device)
        assert hip.mm_from_float(left.to(hip_device), right.to(hip_device), cfg, status=status,
                                 mailbox=box) is not None
        flags = hip.status_wait(box)
        assert flags is not None and flags & checks == bits
        if not bits:
            assert flags == 0
        torch.cuda.synchronize()
        assert int(status.item()) & checks == bits


def range_flag(cfg, peak, device, box, n=64, k=256, o=128):
    """STATUS_RANGE of mm_from_float on saturating operands (every code at its extreme, every
    group scale peak / 127; row 0 of A and column 0 of B all positive, so output (0, 0) is
    the largest product the codes allow), and the call's output."""
    signs_a = torch.randn(n, k, generator=torch.Generator().manual_seed(1)).sign()
    signs_b = torch.randn(k, o, generator=torch.Generator().manual_seed(2)).sign()
    signs_a[0], signs_b[:, 0] = 1.0, 1.0
    a, b = signs_a * peak, signs_b * peak
    fused = hip.mm_from_float(a.to(device), b.to(device), cfg, status=hip.status_word(device),
                              mailbox=box)
    flags = hip.status_wait(box)
    assert flags is not None and not flags & (hip.STATUS_INPUT | hip.STATUS_WEIGHT)
    return bool(flags & hip.STATUS_RANGE), a, b, fused[3]


def test_range_flag_bounds_the_fp32_restore(hip_device):
    """Below the scale at which the quantizers set STATUS_RANGE no FP32 step of the read's
    restore can overflow: worst-case operands (every code saturated, the largest |total| of
    every read) just below it give finite outputs equal to the oracle's.  The threshold is
    found by bisection on the device; it is far above ordinary data, and Simulator.mm above
    it reads the status word after the read (FP64 retry or the reference's error)."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    box = hip.mailbox()
    lo, hi = 1.0, 1e38                     # no flag at lo, flag at hi
    assert not range_flag(cfg, lo, hip_device, box)[0] and range_flag(cfg, hi, hip_device, box)[0]
    while hi / lo > 1.0001:
        mid = math.sqrt(lo * hi)
        if range_flag(cfg, mid, hip_device, box)[0]:
            hi = mid
        else:
            lo = mid
    say("range threshold (peak)", lo)
    flagged, a, b, out = range_flag(cfg, lo, hip_device, box)
    assert not flagged
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert bits_equal(out, oracle.mm(a, b, cfg))
    # The worst-case output at the threshold is within 2^8 of FP32's range: the bound
    # leaves no needless fallback for data that fits.
    assert float(out.abs().max()) > torch.finfo(torch.float32).max / 256
    sim = Simulator(cfg, device=hip_device)
    for scale in (hi * 1.01, 1e30):
        flagged, a, b, _ = range_flag(cfg, scale, hip_device, box)
        assert flagged
        expected = None
        try:
            expected = oracle.mm(a, b, cfg)
        except FloatingPointError:
            pass
        if expected is None or not torch.isfinite(expected).all():
            with pytest.raises(FloatingPointError):
                sim.mm(a.to(hip_device), b.to(hip_device))
        else:
            assert bits_equal(sim.mm(a.to(hip_device), b.to(hip_device)), expected)


def test_pipelined_products_keep_their_results(hip_device):
    """Simulator.mm on the fused route returns once the quantizers' status is published, and
    the read finishes behind the caller's next work.  Consecutive products of one shape (each
    writes the codes and scales of the last one again), one on a side stream (which gets its
    own scratch), one with a bf16 output and one that overflows FP32 (full status read, FP64
    retry) all equal the oracle's."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(12)
    n, k, o = 256, 1024, 512
    pairs = [(torch.randn(n, k, generator=gen), torch.randn(k, o, generator=gen))
             for _ in range(4)]
    big = (torch.randn(n, k, generator=gen) * 1e37, torch.randn(k, o, generator=gen) * 1e-8)
    sim = Simulator(cfg, device=hip_device)
    assert hip.from_float_applies(cfg, n, k, o)
    outs = [sim.mm(a.to(hip_device), b.to(hip_device)) for a, b in pairs[:2]]
    main = torch.cuda.current_stream(hip_device)
    side = torch.cuda.Stream(device=hip_device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        a, b = pairs[2]
        outs.append(sim.mm(a.to(hip_device), b.to(hip_device)))
    main.wait_stream(side)
    a, b = pairs[3]
    outs.append(sim.mm(a.to(hip_device).bfloat16(), b.to(hip_device).bfloat16()))
    overflow = sim.mm(big[0].to(hip_device), big[1].to(hip_device))
    torch.cuda.synchronize()
    for i, ((a, b), got) in enumerate(zip(pairs, outs)):
        if i == 3:
            a, b = a.bfloat16(), b.bfloat16()
        assert bits_equal(got, oracle.mm(a, b, cfg)), i
    expected = oracle.mm(*big, cfg)
    assert torch.isfinite(expected).all() and bits_equal(overflow, expected)


def test_mm_from_float_declines_other_shapes(hip_device):
    """Shapes and configurations outside the fused route launch nothing and return None;
    Simulator.mm then takes the separate calls (checked against the oracle)."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    cases = [(cfg, 8, 150, 128), (cfg, 8, 256, 100),
             (ideal(**CONFIG2 | dict(input_quant_gran=(1, None))), 8, 256, 128),
             (Config(**CONFIG2, nonidealities=Nonidealities(write_variation=0.02)), 8, 256, 128)]
    for config, n, k, o in cases:
        assert not hip.from_float_applies(config, n, k, o)
        a, b = torch.randn(n, k), torch.randn(k, o)
        assert hip.mm_from_float(a.to(hip_device), b.to(hip_device), config) is None
        if config.nonidealities.write_variation == 0.0:
            got = Simulator(config, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
            assert bits_equal(got, oracle.mm(a, b, config))


def test_functional_nonfinite_operands_leave_simulator_unchanged(hip_device):
    """The fused product checks finiteness on the device (functional.py:49-53 order)."""
    from memfast_amd import Simulator, mm

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(5)
    a = torch.randn(6, 256, generator=gen)
    b = torch.randn(256, 40, generator=gen)
    sim = Simulator(cfg, device=hip_device)
    bad_a, bad_b = a.clone(), b.clone()
    bad_a[3, 100] = float("nan")
    bad_b[7, 2] = float("inf")
    cases = [(bad_a, b, "A must be finite"), (a, bad_b, "B must be finite"),
             (bad_a, bad_b, "A must be finite")]
    for left, right, message in cases:
        with pytest.raises(ValueError, match=message):
            sim.mm(left.to(hip_device), right.to(hip_device))
        with pytest.raises(ValueError, match=message):
            mm(left.to(hip_device).bfloat16(), right.to(hip_device).bfloat16(), config=cfg)
    assert sim._next_id == 0 and not sim._matrix_cache
    assert bits_equal(sim.mm(a.to(hip_device), b.to(hip_device)), oracle.mm(a, b, cfg))


def test_unsigned_weight_error_follows_finiteness_errors(hip_device):
    """Unsigned configurations: a non-finite A (or B) raises its finiteness error before a
    negative weight raises the unsigned-weight error, as memfast/functional.py:51-53 checks
    finiteness before memfast/quantization.py:14-18 quantizes; narrow and wide."""
    from memfast_amd import Simulator

    for cfg in (ideal(weight_bits=4, weight_signed=False, weight_slice=(2, 2),
                      array_size=(32, 16), adc_bits=5),
                ideal(activation_bits=12, weight_bits=10, weight_signed=False,
                      array_size=(32, 16), adc_bits=8)):
        gen = torch.Generator().manual_seed(8)
        a, b = torch.randn(4, 40, generator=gen), torch.randn(40, 20, generator=gen).abs()
        bad_a, negative_b, bad_b = a.clone(), -b, b.clone()
        bad_a[1, 3] = float("nan")
        bad_b[2, 2] = float("inf")
        negative_bad_b = negative_b.clone()
        negative_bad_b[2, 2] = float("nan")
        sim = Simulator(cfg, device=hip_device)
        cases = [(bad_a, negative_b, "A must be finite"), (a, negative_bad_b, "B must be finite"),
                 (a, negative_b, "unsigned floating weights must be nonnegative"),
                 (bad_a, bad_b, "A must be finite")]
        for left, right, message in cases:
            with pytest.raises(ValueError, match=message):
                sim.mm(left.to(hip_device), right.to(hip_device))
        assert sim._next_id == 0
        assert bits_equal(sim.mm(a.to(hip_device), b.to(hip_device)), oracle.mm(a, b, cfg))


def test_functional_reprogramming_follows_in_place_edits(hip_device):
    """Reused RHS programs take new codes in place and keep name and event counter."""
    from memfast_amd import Simulator

    cfg = Config(**SMALL, nonidealities=Nonidealities(write_variation=0.0, read_variation=0.01))
    gen = torch.Generator().manual_seed(6)
    a = torch.randn(5, 256, generator=gen)
    b = torch.randn(256, 40, generator=gen)
    sim = Simulator(cfg, device=hip_device)
    a_dev, b_dev = a.to(hip_device), b.to(hip_device)
    outputs = [sim.mm(a_dev, b_dev)]
    program = sim._matrix_cache.program(b_dev)
    b_dev.mul_(-0.5)
    outputs.append(sim.mm(a_dev, b_dev))
    assert sim._matrix_cache.program(b_dev) is program and program._event == 2
    assert program.name == "matrix.0" and sim._next_id == 1
    for event, (weights, got) in enumerate(zip((b, b * -0.5), outputs)):
        check_product(cfg, got, a, weights, hip_device, event=event, label=f"event {event}")


def test_fp32_overflow_retries_in_fp64(hip_device):
    """Non-finite FP32 restores repeat in FP64 (simulator.py:614-615); FP64 operands keep it."""
    from memfast_amd import Simulator

    cfg = ideal(**CONFIG2)
    gen = torch.Generator().manual_seed(7)
    a = torch.randn(4, 256, generator=gen, dtype=torch.float64) * 1e30
    b = torch.randn(256, 36, generator=gen, dtype=torch.float64) * 1e30
    sim = Simulator(cfg, device=hip_device)
    got = sim.mm(a.to(hip_device), b.to(hip_device))
    expected = oracle.mm(a, b, cfg)
    assert got.dtype == torch.float64 and torch.isfinite(got).all()
    assert bits_equal(got, expected)
    with pytest.raises(FloatingPointError):
        sim.mm(a.float().to(hip_device), b.float().to(hip_device))


@pytest.mark.parametrize("name", ["int12_ideal", "bfp16_int4"])
def test_wide_product_cast_flags_nonfinite_outputs(hip_device, name):
    """A wide product of FP32 operands casts its FP64 restore to FP32 on the device
    (mf_narrow_output) and flags a non-finite result in the status word: the outputs equal
    torch's cast of the same product of the FP64 operands bit for bit, and a cast that
    overflows raises FloatingPointError (memfast/simulator.py:642-644) where the FP64
    product stays finite.  Layer reads of FP32 inputs cast the same way."""
    from memfast_amd import Simulator

    cfg = wide_case(name)
    gen = torch.Generator().manual_seed(48)
    a = torch.randn(37, 150, generator=gen)
    b = torch.randn(150, 70, generator=gen)
    got = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    wide = Simulator(cfg, device=hip_device).mm(a.double().to(hip_device),
                                                 b.double().to(hip_device))
    assert got.dtype == torch.float32 and wide.dtype == torch.float64
    assert bits_equal(got, wide.float())
    big_a, big_b = (a * 1e30).to(hip_device), (b * 1e30).to(hip_device)
    sim = Simulator(cfg, device=hip_device)
    assert torch.isfinite(sim.mm(big_a.double(), big_b.double())).all()
    with pytest.raises(FloatingPointError):
        sim.mm(big_a, big_b)
    again = sim.mm(a.to(hip_device), b.to(hip_device))
    # (noise is keyed by the program's name and event, which the earlier calls moved on)
    assert torch.isfinite(again).all() and (name != "int12_ideal" or bits_equal(again, got))
    # A layer read (bias included) casts the same way.
    from torch import nn

    from memfast_amd.nn import AnalogLinear

    source = nn.Linear(150, 70).to(hip_device)
    layers = [AnalogLinear(source, Simulator(cfg, device=hip_device), name="cast")
              for _ in range(2)]
    x = a.to(hip_device)
    with torch.no_grad():
        narrow, full = layers[0](x), layers[1](x.double())
    assert narrow.dtype == torch.float32 and bits_equal(narrow, full.float())


def test_wide_range_flag_and_early_status(hip_device, monkeypatch):
    """Wide quantizers flag STATUS_RANGE for a group scale above
    s = sqrt(FLT_MAX / (2 * G * Config.reconstruction_bound)) (G reads), the bound under
    which the FP64 restore cast to FP32 stays below FLT_MAX / 2.  Without the flag, a wide
    product returns on the quantizers' bits, published before the read: its outputs equal
    the full status read's bit for bit; with it the product reads the device word and
    raises FloatingPointError where the cast overflows."""
    from memfast_amd import Simulator

    cfg = wide_case("int12_ideal")
    k = 150
    G = -(-k // cfg.array_size[0]) * cfg.reads_per_array
    s = math.sqrt(torch.finfo(torch.float32).max / (2 * G * cfg.reconstruction_bound))
    upper = 2 ** (cfg.activation_bits - 1) - 1
    for factor, flagged in ((0.99, False), (1.01, True)):
        a = torch.zeros(3, k, device=hip_device)
        a[:, 5] = s * factor * upper   # group scale = peak / upper
        status = hip.status_word(hip_device)
        hip.input_tiles(a, cfg, status=status)
        assert bool(int(status.item()) & hip.STATUS_RANGE) == flagged, factor
    gen = torch.Generator().manual_seed(49)
    a = torch.randn(37, k, generator=gen).to(hip_device)
    b = torch.randn(k, 70, generator=gen).to(hip_device)
    seen = []
    wait = hip.status_wait

    def spy(box, timeout_s=10.0):
        seen.append(wait(box, timeout_s))
        return seen[-1]

    monkeypatch.setattr(hip, "status_wait", spy)
    early = Simulator(cfg, device=hip_device).mm(a, b)
    assert seen == [0]
    monkeypatch.setattr(hip, "status_wait", lambda box, timeout_s=10.0: None)
    full = Simulator(cfg, device=hip_device).mm(a, b)
    assert bits_equal(early, full)
    monkeypatch.setattr(hip, "status_wait", spy)
    with pytest.raises(FloatingPointError):
        Simulator(cfg, device=hip_device).mm(a * 1e30, b * 1e30)
    assert seen[-1] is not None and seen[-1] & hip.STATUS_RANGE


@pytest.mark.parametrize("groups,width,c", [(5, 1, 4), (17, 2, 12), (128, 2, 128), (300, 1, 36),
                                            (40, 2, 4)])
def test_stable_sum_matches_cpu_restore(hip_device, groups, width, c):
    """FP64 restore + read sum equals oracle.restore_scales(...).sum(1) on the CPU, bit for bit."""
    cfg = ideal(**CONFIG2 | dict(array_size=(128, c)))
    gen = torch.Generator().manual_seed(groups * 7 + c)
    n = 3
    totals = torch.randint(-5000, 5000, (n, groups, width, c), generator=gen).float()
    xs = torch.exp(15 * torch.randn(n, groups, generator=gen)).float()
    ws = torch.exp(15 * torch.randn(groups, width * c, generator=gen)).float()
    expected = oracle.restore_scales(totals, xs[:, :, None, None],
                                     ws.reshape(groups, width, c)[None]).sum(1).flatten(1)
    # The chunk sits at columns [8, 8 + width*C) of the output and of the scale rows.
    out = torch.zeros((n, width * c + 8), dtype=torch.float64, device=hip_device)
    ws_rows = torch.cat([torch.ones(groups, 8), ws], dim=1)
    hip.stable_sum(totals.to(hip_device), xs.to(hip_device), ws_rows.to(hip_device), cfg, 8, out)
    assert bits_equal(out[:, 8:], expected)


# ---------------------------------------------------------------------------
# Noisy devices on the fp16 MFMA kernel (hi + lo terms; reads of 32 or 64 rows)
# ---------------------------------------------------------------------------
MFMA_NOISY = {
    "write": (dict(), dict(write_variation=0.02)),
    "shared_scurve": (dict(), dict(write_variation=0.02, read_variation=0.01,
                                   adc_nonlinearity=0.1)),
    "saf_drift": (dict(), dict(write_variation=0.02, stuck_at_low=0.05, stuck_at_high=0.03,
                               drift_coefficient=0.05, drift_time=100.0)),
    "binary8": (dict(input_slice=None, weight_slice=(1, 1, 2, 2, 2), adc_bits=(4, 5, 5, 6, 6)),
                dict(write_variation=0.03, adc_nonlinearity=0.05)),
    "rows64": (dict(array_size=(128, 32), rows_per_read=64, weight_quant_gran=(64, 1),
                    input_quant_gran=(1, 64)), dict(write_variation=0.02, read_variation=0.01)),
    # Voltage variation: real input operands (hi + lo), 2-bit and binary digits, 32- and
    # 64-row reads, with shared read noise and the S-curve ADC.
    "voltage": (dict(), dict(write_variation=0.02, voltage_variation=0.05)),
    "voltage_binary8": (dict(input_slice=None, weight_slice=(1, 1, 2, 2, 2),
                             adc_bits=(4, 5, 5, 6, 6)),
                        dict(write_variation=0.02, voltage_variation=0.03)),
    "voltage_rows64": (dict(array_size=(128, 32), rows_per_read=64, weight_quant_gran=(64, 1),
                            input_quant_gran=(1, 64)),
                       dict(write_variation=0.02, read_variation=0.01, voltage_variation=0.02,
                            adc_nonlinearity=0.1)),
    # slice_pair read noise: one plane of conductance terms per input slice; with binary
    # digits (8 planes), and at 64-row reads with voltage noise and the S-curve.
    "slice_pair": (dict(), dict(write_variation=0.02, read_variation=0.02,
                                read_mode="slice_pair")),
    "slice_pair_binary8": (dict(input_slice=None, weight_slice=(1, 1, 2, 2, 2),
                                adc_bits=(4, 5, 5, 6, 6)),
                           dict(write_variation=0.02, read_variation=0.02,
                                read_mode="slice_pair")),
    "slice_pair_rows64": (dict(array_size=(128, 32), rows_per_read=64,
                               weight_quant_gran=(64, 1), input_quant_gran=(1, 64)),
                          dict(write_variation=0.02, read_variation=0.01, read_mode="slice_pair",
                               voltage_variation=0.02, adc_nonlinearity=0.1)),
    # Output-mode read noise: mean and variance sums beside the current, one normal per
    # conversion; with binary digits, and at 64-row reads with SAF and the S-curve.
    "output": (dict(), dict(write_variation=0.02, read_variation=0.02, read_mode="output")),
    "output_binary8": (dict(input_slice=None, weight_slice=(1, 1, 2, 2, 2),
                            adc_bits=(4, 5, 5, 6, 6)),
                       dict(write_variation=0.02, read_variation=0.03, read_mode="output")),
    "output_rows64": (dict(array_size=(128, 32), rows_per_read=64, weight_quant_gran=(64, 1),
                           input_quant_gran=(1, 64)),
                      dict(write_variation=0.02, read_variation=0.02, read_mode="output",
                           stuck_at_low=0.01, stuck_at_high=0.01, adc_nonlinearity=0.1)),
    # Output-mode read noise with voltage variation: real operands x and x*x (hi + lo) for
    # the current and variance sums; 2-bit and binary digits, 32- and 64-row reads.
    "output_voltage": (dict(), dict(write_variation=0.02, read_variation=0.02,
                                    read_mode="output", voltage_variation=0.05)),
    "output_voltage_binary8": (dict(input_slice=None, weight_slice=(1, 1, 2, 2, 2),
                                    adc_bits=(4, 5, 5, 6, 6)),
                               dict(write_variation=0.02, read_variation=0.03, read_mode="output",
                                    voltage_variation=0.03, adc_nonlinearity=0.1)),
    "output_voltage_rows64": (dict(array_size=(128, 32), rows_per_read=64,
                                   weight_quant_gran=(64, 1), input_quant_gran=(1, 64)),
                              dict(write_variation=0.02, read_variation=0.02, read_mode="output",
                                   voltage_variation=0.02)),
}
NOISY_BASE = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                  weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                  weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))


def noisy_case(mode):
    extra, effects = MFMA_NOISY[mode]
    return Config(**(NOISY_BASE | extra), nonidealities=Nonidealities(**effects))


def packed_columns(packed):
    m, p, r, c = packed.shape
    return packed.permute(1, 3, 0, 2).reshape(p * c, m * r).contiguous()


@pytest.mark.parametrize("mode", ["write", "shared_scurve", "saf_drift", "binary8", "rows64"])
def test_small_batch_split_read_matches_unsplit_read(hip_device, mode):
    """Batches of at most 32 vectors split their reads over k_noisy_pairs (one workgroup per
    read and 32-column block, one wave per weight slice; the restored values are summed by
    the split epilogue).  Every schedule (automatic, unsplit k_noisy, a 2-way split) gives
    the same output bit for bit: 32- and 64-row reads, 5 and 8 input slices, S-curve ADCs;
    and the product is the oracle's under the flip accounting."""
    cfg = noisy_case(mode)
    gen = torch.Generator().manual_seed(34)
    for n in (1, 7, 32):
        a = torch.randn(n, 500, generator=gen)
        b = torch.randn(500, 300, generator=gen)
        q, xs = hip.input_tiles(a.to(hip_device), cfg)
        packed, packed_t, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
        m, p, c = q.shape[1], packed.shape[1], cfg.array_size[1]
        assert hip.mm_kernel(cfg, n, m, p) == 2
        outputs = [hip.mm(q, xs, packed, packed_t, ws.reshape(-1, p * c), cfg, 4242, 3,
                          variant=hip.variant_word(split=split)) for split in (0, 1, 2)]
        say("  small batch", mode, n, "automatic, 2-way split vs unsplit",
            bits_equal(outputs[0], outputs[1]), bits_equal(outputs[2], outputs[1]))
        assert bits_equal(outputs[0], outputs[1]) and bits_equal(outputs[2], outputs[1])
    from memfast_amd import Simulator

    got = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    check_product(cfg, got, a, b, hip_device, label=f"small batch {mode}")


@pytest.mark.parametrize("mode", list(MFMA_NOISY))
def test_noisy_mfma_totals_with_injected_conductances(hip_device, mode):
    """Same slice totals as the oracle given the same conductances, except ADC flips."""
    say("noisy mfma totals", mode)
    cfg = noisy_case(mode)
    gen = torch.Generator().manual_seed(31)
    a = torch.randn(40, 200, generator=gen)
    b = torch.randn(200, 100, generator=gen)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    n, m, r = q.shape
    p = packed.shape[1]
    assert hip.mm_kernel(cfg, n, m, p) == 2
    seed, event = 4242, 3
    raw, _, _ = oracle.restored(packed, cfg, seed, event, 0, p)
    expected = oracle.partial(q, packed, cfg, seed, event, 0, p, conductance=raw)
    got = hip.mm_totals(q.to(hip_device), packed_columns(packed).to(hip_device), cfg, seed, event,
                        conductance=raw.to(hip_device)).cpu()
    diff = got.double() - expected.double()
    codes = diff.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    flips = int((diff != 0).sum())
    largest = max(abs(fa * fw) for _, _, fa in cfg.input_layout for _, _, fw in cfg.weight_layout)
    say("  totals differing", flips, "of", diff.numel(), "max", diff.abs().max().item())
    assert flips <= max(1, 1e-4 * codes)
    assert diff.abs().max().item() <= 2 * largest


@pytest.mark.parametrize("mode", list(MFMA_NOISY))
def test_noisy_mfma_sampled_conductances(hip_device, mode):
    """Conductances sampled on the GPU (counter RNG, OCML) against the oracle's samples."""
    cfg = noisy_case(mode)
    gen = torch.Generator().manual_seed(32)
    a = torch.randn(40, 200, generator=gen)
    b = torch.randn(200, 100, generator=gen)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    p = packed.shape[1]
    seed, event = 99, 7
    expected = oracle.partial(q, packed, cfg, seed, event, 0, p)
    got = hip.mm_totals(q.to(hip_device), packed_columns(packed).to(hip_device), cfg, seed,
                        event).cpu()
    diff = got.double() - expected.double()
    codes = diff.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    flips = int((diff != 0).sum())
    say("  totals differing", flips, "of", diff.numel())
    assert flips <= max(1, 1e-4 * codes)


@pytest.mark.parametrize("mode", list(MFMA_NOISY))
def test_noisy_mfma_epilogue_and_mm(hip_device, mode):
    """Fused output = the reference epilogue of the kernel's own totals, bit for bit; and
    Simulator.mm within the flip budget of the oracle."""
    from memfast_amd import Simulator

    cfg = noisy_case(mode)
    gen = torch.Generator().manual_seed(33)
    a = torch.randn(40, 200, generator=gen)
    b = torch.randn(200, 100, generator=gen)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    seed, event = 1234, 0
    codes_t = packed_columns(packed).to(hip_device)
    totals = hip.mm_totals(q.to(hip_device), codes_t, cfg, seed, event).cpu()
    fused = hip.mm(q.to(hip_device), xs.to(hip_device), packed.to(hip_device), codes_t,
                   ws.reshape(-1, p * c).to(hip_device), cfg, seed, event).cpu()
    restored = oracle.execute(q, xs, packed, ws, cfg, seed, event, p * c, totals=totals)
    assert bits_equal(fused, restored)
    sim = Simulator(cfg, device=hip_device)
    got = sim.mm(a.to(hip_device), b.to(hip_device))
    check_product(cfg, got, a, b, hip_device, label=f"mfma {mode}")


# ---------------------------------------------------------------------------
# Wide configurations (precision above 8 bits, BFP): FP64 scales and restore
# ---------------------------------------------------------------------------
WIDE = {
    "bfp16_int4": (dict(activation_bits=16, weight_bits=4,
                        input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2), weight_slice=(1, 1, 2), bw_e=8,
                        array_size=(64, 64), adc_bits=(6, 6, 7)),
                   dict(write_variation=0.02, read_variation=0.01, drift_coefficient=0.05,
                        drift_time=100.0)),
    "int12_ideal": (dict(activation_bits=12, weight_bits=10, array_size=(32, 16),
                         rows_per_read=16, adc_bits=8), dict(write_variation=0.0)),
    "bfp8_binary": (dict(activation_bits=8, weight_bits=8, bw_e=4, array_size=(32, 16),
                         rows_per_read=16, adc_bits=6),
                    dict(write_variation=0.02, adc_nonlinearity=0.05)),
}


def wide_case(name):
    kwargs, effects = WIDE[name]
    return Config(**kwargs, nonidealities=Nonidealities(**effects))


@pytest.mark.parametrize("name", list(WIDE))
def test_wide_tiles_match_reference_vectors(hip_device, reference_vectors, name):
    v = reference_vectors
    cfg = wide_case(name)
    a = torch.from_numpy(v[f"case_{name}_a"]).to(hip_device)
    b = torch.from_numpy(v[f"case_{name}_b"]).to(hip_device)
    q, xs = hip.input_tiles(a, cfg)
    packed, codes, ws = hip.weight_tiles(b.T, cfg)
    torch.cuda.synchronize()
    expected_q = torch.from_numpy(v[f"case_{name}_q"]).to(torch.int64)
    assert bits_equal(q.cpu().to(torch.int64) & 0xFFFFFFFF, expected_q)
    assert bits_equal(xs, torch.from_numpy(v[f"case_{name}_xscale"]))
    expected_packed = torch.from_numpy(v[f"case_{name}_packed"])
    assert packed.dtype == expected_packed.dtype
    assert bits_equal(packed, expected_packed)
    assert bits_equal(codes.cpu().to(torch.int64) & 0xFFFFFFFF, expected_packed.to(torch.int64))
    assert bits_equal(ws, torch.from_numpy(v[f"case_{name}_wscale"]))


@pytest.mark.parametrize("name", list(WIDE))
def test_wide_totals_with_injected_conductances(hip_device, reference_vectors, name):
    v = reference_vectors
    cfg = wide_case(name)
    q = torch.from_numpy(v[f"case_{name}_q"]).to(hip_device)
    packed = torch.from_numpy(v[f"case_{name}_packed"]).to(hip_device)
    seed = int(v[f"case_{name}_seed"])
    p = packed.shape[1]
    raw = torch.from_numpy(v[f"case_{name}_restored"]).to(hip_device)
    totals = hip.partial(q, packed, cfg, None, seed, 0, 0, p, conductance=raw).cpu()
    expected = torch.from_numpy(v[f"case_{name}_totals"])
    assert totals.dtype == torch.float64
    diff = totals - expected
    codes = diff.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    say("  wide totals differing", int((diff != 0).sum()), "of", diff.numel())
    if cfg.nonidealities.ideal:
        assert bits_equal(totals, expected)
    else:
        assert int((diff != 0).sum()) <= max(1, 1e-4 * codes)


@pytest.mark.parametrize("name", list(WIDE))
def test_wide_mm_matches_reference_vectors(hip_device, reference_vectors, name):
    from memfast_amd import Simulator

    v = reference_vectors
    cfg = wide_case(name)
    a = torch.from_numpy(v[f"case_{name}_a"]).to(hip_device)
    b = torch.from_numpy(v[f"case_{name}_b"]).to(hip_device)
    sim = Simulator(cfg, device=hip_device)
    q = torch.from_numpy(v[f"case_{name}_q"])
    packed = torch.from_numpy(v[f"case_{name}_packed"])
    xs = torch.from_numpy(v[f"case_{name}_xscale"])
    ws = torch.from_numpy(v[f"case_{name}_wscale"])
    seed = int(v[f"case_{name}_seed"])
    for event in (0, 1):
        got = sim.mm(a, b)
        ref = torch.from_numpy(v[f"case_{name}_out{event}"])
        if cfg.nonidealities.ideal:
            assert bits_equal(got, ref)
            continue
        totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, event)
        if event == 0:
            ref_totals = torch.from_numpy(v[f"case_{name}_totals"])
        else:
            ref_totals = oracle_totals(q, packed, cfg, seed, event)
            ref = oracle.execute(q, xs, packed, ws, cfg, seed, event, b.shape[1],
                                 totals=ref_totals).float()
        say("  wide", name, "event", event,
            flips.check_noisy(cfg, got, ref, totals, ref_totals, xscale=xs, wscale=ws,
                              label=f"wide {name} event {event}"))


def test_bfp_exponent_edges_on_gpu(hip_device, reference_vectors):
    """BFP scales and codes at power-of-two group maxima (quantization.py:35-40)."""
    v = reference_vectors
    edges = torch.from_numpy(v["bfp_edges_in"])
    for bits, bw_e in ((16, 8), (12, 5), (8, 11)):
        cfg = Config(activation_bits=bits, weight_bits=4, bw_e=bw_e, array_size=(4, 4),
                     input_quant_gran=(1, 4), adc_bits=4)
        q, xs = hip.input_tiles(edges.to(hip_device), cfg)
        codes = torch.from_numpy(v[f"bfp_edges_code_{bits}_{bw_e}"]) & ((1 << bits) - 1)
        scales = torch.from_numpy(v[f"bfp_edges_scale_{bits}_{bw_e}"])
        assert bits_equal(q.reshape(edges.shape).cpu().to(torch.int64) & 0xFFFFFFFF, codes)
        assert bits_equal(xs[:, 0].cpu(), scales[:, 0])


# ---------------------------------------------------------------------------
# FP64 currents (memfast/config.py:215-224 `precise_currents`): k_restore<double> and
# k_general<double> against the reference's own vectors (tests/golden)
# ---------------------------------------------------------------------------
PRECISE = ["precise_slice9_ideal", "precise_slice9", "precise_close_ideal", "precise_close"]


def _precise_case(v, name, device):
    from conftest import fixture_config

    cfg = fixture_config(v, name)
    assert cfg.precise_currents
    q = torch.from_numpy(v[f"case_{name}_q"])
    packed = torch.from_numpy(v[f"case_{name}_packed"])
    assert hip.mm_kernel(cfg, q.shape[0], q.shape[1], packed.shape[1]) == 0
    return cfg, q, packed, int(v[f"case_{name}_seed"])


def _pair_codes_closed_form(q, packed, cfg):
    """Ideal ADC counts min(sum_r da*dw, max_w) per pair, [N, m*Gr, A, W, p*C]."""
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    rows, groups = cfg.read_rows, cfg.reads_per_array
    maxima = cfg.adc_maxima
    out = torch.zeros((n, m * groups, len(cfg.input_layout), len(cfg.weight_layout), p * c),
                      dtype=torch.int64)
    for ai, (sa, ma, _) in enumerate(cfg.input_layout):
        da = (q.long() >> sa) & ma
        for wi, (sw, mw, _) in enumerate(cfg.weight_layout):
            dw = (packed.long() >> sw) & mw
            for j in range(groups):
                lo, hi = j * rows, min((j + 1) * rows, r)
                s = torch.einsum("nir,itrc->nitc", da[:, :, lo:hi], dw[:, :, lo:hi])
                out[:, j::groups, ai, wi] = s.clamp_max(maxima[wi]).reshape(n, m, p * c)
    return out


@pytest.mark.parametrize("name", PRECISE)
def test_precise_partial_matches_reference_vectors(hip_device, reference_vectors, name):
    """mf_partial's totals (k_general<double>) against the reference's at its seed and event:
    bit for bit with ideal devices, where every per-pair ADC count is also the closed form
    min(sum_r da*dw, max_w); with noise, given the reference's own FP64 conductances, identical
    except rounding-boundary flips."""
    v = reference_vectors
    cfg, q, packed, seed = _precise_case(v, name, hip_device)
    p = packed.shape[1]
    reference = torch.from_numpy(v[f"case_{name}_totals"])
    if cfg.nonidealities.ideal:
        got, codes = hip.partial(q.to(hip_device), packed.to(hip_device), cfg, None, seed, 0, 0,
                                 p, codes=True)
        assert bits_equal(got, reference)
        assert torch.equal(codes.cpu().long(), _pair_codes_closed_form(q, packed, cfg))
        return
    raw = torch.from_numpy(v[f"case_{name}_restored"])
    assert raw.dtype == torch.float64
    got = hip.partial(q.to(hip_device), packed.to(hip_device), cfg, None, seed, 0, 0, p,
                      conductance=raw.to(hip_device))
    differing, flipped, unexplained, mask = flips.count_flips(cfg, got.cpu(), reference)
    codes = mask.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    say("  precise", name, "injected:", differing, "differing totals,", flipped, "flips of", codes)
    assert unexplained == 0
    assert flipped <= max(1, 1e-4 * codes)


@pytest.mark.parametrize("name", ["precise_slice9", "precise_close"])
def test_precise_restore_close_to_reference(hip_device, reference_vectors, name):
    """k_restore<double>: FP64 conductances with write and shared read noise against the
    reference's restored tensor (same seed, event 0)."""
    v = reference_vectors
    cfg, q, packed, seed = _precise_case(v, name, hip_device)
    got = hip.restore(packed.to(hip_device), cfg, seed, 0, 0, packed.shape[1])
    assert got.dtype == torch.float64 and got.shape[0] == 1
    expected = torch.from_numpy(v[f"case_{name}_restored"])
    # The noise factors are FP32 (torch.exp of an FP32 normal); OCML's and torch CPU's
    # transcendentals agree to an ulp or two of the factor (2.4e-7 relative).
    ratio = got[0].cpu() / expected - 1
    assert float(ratio.abs().max()) <= 2.4e-7


@pytest.mark.parametrize("name", PRECISE)
def test_precise_mm_matches_reference_vectors(hip_device, reference_vectors, name):
    """Simulator.mm with FP64 currents for two read events against the reference's outputs:
    bit for bit with ideal devices, flip-aware with noise (GPU-sampled conductances).

    With high - low = 5e-5 of high (precise_close), one FP32 ulp of a noise factor moves g by
    0.24% of high - low, so sampled codes are only as reproducible as the host's FP32
    exp/log/cos: the reference's own restored tensor differs between two x86 hosts (this
    test's and the fixture's).  There the bar is the injected one
    (test_precise_partial_matches_reference_vectors), and the sampled product is checked
    to be that read of its own samples: its totals equal mf_partial's with the GPU's restored
    conductances injected, and its output is the reference epilogue of those totals."""
    from memfast_amd import Simulator

    v = reference_vectors
    cfg, q, packed, seed = _precise_case(v, name, hip_device)
    a = torch.from_numpy(v[f"case_{name}_a"]).to(hip_device)
    b = torch.from_numpy(v[f"case_{name}_b"]).to(hip_device)
    xs = torch.from_numpy(v[f"case_{name}_xscale"])
    ws = torch.from_numpy(v[f"case_{name}_wscale"])
    sim = Simulator(cfg, device=hip_device)
    for event in (0, 1):
        got = sim.mm(a, b)
        ref = torch.from_numpy(v[f"case_{name}_out{event}"])
        if cfg.nonidealities.ideal:
            assert bits_equal(got, ref)
            continue
        totals = gpu_totals(q.to(hip_device), packed.to(hip_device), cfg, seed, event)
        if name == "precise_close":
            p = packed.shape[1]
            own = hip.restore(packed.to(hip_device), cfg, seed, event, 0, p)
            injected = hip.partial(q.to(hip_device), packed.to(hip_device), cfg, None, seed,
                                   event, 0, p, conductance=own)
            assert bits_equal(totals, injected)
            epilogue = oracle.execute(q, xs, packed, ws, cfg, seed, event, b.shape[1],
                                      totals=totals.cpu().to(injected.dtype)).to(got.dtype)
            assert bits_equal(got, epilogue)
            continue
        if event == 0:
            ref_totals = torch.from_numpy(v[f"case_{name}_totals"])
        else:
            ref_totals = oracle_totals(q, packed, cfg, seed, event)
            ref = oracle.execute(q, xs, packed, ws, cfg, seed, event, b.shape[1],
                                 totals=ref_totals).to(ref.dtype)
        say("  precise", name, "event", event,
            flips.check_noisy(cfg, got, ref, totals, ref_totals, xscale=xs, wscale=ws,
                              label=f"precise {name} event {event}"))


PRECISE_MFMA = {
    # A 9-bit input digit (mask 511 > 255): FP64 currents.  Write and shared read noise with
    # the S-curve ADC; ideal devices; slice_pair read noise (one plane per input slice).
    "slice9": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 2, 9),
                    weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=16,
                    adc_bits=8), dict(write_variation=0.02, read_variation=0.01,
                                      adc_nonlinearity=0.1)),
    "slice9_ideal": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 2, 9),
                          weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                          adc_bits=8), dict(write_variation=0.0)),
    "slice9_pair": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 2, 9),
                         weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=64,
                         adc_bits=8), dict(write_variation=0.02, read_variation=0.02,
                                           read_mode="slice_pair")),
    # High - low = 5e-5 of high, narrow codes; drift and stuck-at faults; 128-row reads.
    "close": (dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                   weight_slice=(1, 1, 2, 2, 2), array_size=(128, 64), rows_per_read=128,
                   adc_bits=(6, 7, 7, 8, 8), high_conductance=1e-5, low_conductance=9.9995e-6),
              dict(write_variation=2e-6, stuck_at_low=0.01, stuck_at_high=0.01,
                   drift_coefficient=0.05, drift_time=100.0)),
    "close_ideal": (dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                         weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                         adc_bits=(6, 7, 7, 8, 8), high_conductance=1e-5,
                         low_conductance=9.9995e-6), dict(write_variation=0.0)),
}


@pytest.mark.parametrize("name", list(PRECISE_MFMA))
def test_precise_mfma_read_matches_general_kernel(hip_device, name):
    """FP64 currents on FP64 MFMA (k_general_mfma64, what Simulator.mm and mf_partial's totals
    run) against k_general<double> (mf_partial with per-pair codes, the reference's
    arithmetic order) on the same conductances: bit for bit with ideal devices, else
    identical but for rounding-boundary flips.  Simulator.mm's fused output is the oracle's
    epilogue of the MFMA totals, bit for bit, and the oracle checks the product as the other
    parity tests do."""
    from memfast_amd import Simulator

    kwargs, effects = PRECISE_MFMA[name]
    cfg = Config(**kwargs, nonidealities=Nonidealities(**effects))
    assert cfg.precise_currents
    gen = torch.Generator().manual_seed(len(name))
    n, k, o = 37, 2 * cfg.array_size[0] + 9, cfg.array_size[1] + 7
    a, b = torch.randn(n, k, generator=gen), torch.randn(k, o, generator=gen)
    dev = hip_device
    q, xs = hip.input_tiles(a.to(dev), cfg)
    packed, _, ws = hip.weight_tiles(b.T.contiguous().to(dev), cfg)
    m, p = q.shape[1], packed.shape[1]
    assert hip.mm_kernel(cfg, n, m, p) == 0
    seed = oracle.name_seed(cfg.seed, "matrix.0")
    g = None if cfg.nonidealities.ideal else hip.restore(packed, cfg, seed, 0, 0, p)
    mfma = hip.partial(q, packed, cfg, None, seed, 0, 0, p, conductance=g)
    general, _ = hip.partial(q, packed, cfg, None, seed, 0, 0, p, conductance=g, codes=True)
    if cfg.nonidealities.ideal:
        assert bits_equal(mfma, general)
    else:
        differing, flipped, unexplained, mask = flips.count_flips(cfg, mfma.cpu().double(),
                                                                  general.cpu().double())
        codes = mask.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
        say("  precise mfma", name, differing, "differing totals,", flipped, "flips of", codes)
        assert unexplained == 0 and flipped <= max(1, 1e-4 * codes)
    got = Simulator(cfg, device=dev).mm(a.to(dev), b.to(dev))
    q_cpu, xs_cpu = oracle.input_tiles(a, cfg)
    packed_cpu, ws_cpu = oracle.weight_tiles(b.T, cfg)
    epilogue = oracle.execute(q_cpu, xs_cpu, packed_cpu, ws_cpu, cfg, seed, 0, o,
                              totals=mfma.cpu().to(mfma.dtype)).to(got.dtype)
    assert bits_equal(got, epilogue)
    check_product(cfg, got, a, b, dev, label=f"precise mfma {name}")


def test_precise_mfma_resources(hip_device):
    """mf_resources_query reports the FP64 MFMA read for precise currents, and k_general
    where voltage variation keeps them there."""
    cfg = Config(**PRECISE_MFMA["slice9"][0], nonidealities=Nonidealities(write_variation=0.02))
    volt = Config(**PRECISE_MFMA["slice9"][0],
                  nonidealities=Nonidealities(write_variation=0.02, voltage_variation=0.02))
    plain = hip.program(cfg, 64, 64, hip_device.index).resources(cfg, 64, 64, 0, kernel=0)
    general = hip.program(volt, 64, 64, hip_device.index).resources(volt, 64, 64, 0, kernel=0)
    say("precise resources", plain, general)
    assert plain["threads"] == general["threads"] == 256
    assert plain != general


# ---------------------------------------------------------------------------
# Wide configurations on the noisy-device fp16 MFMA kernel (mm_kernel 3)
# ---------------------------------------------------------------------------
WIDE_MFMA = {
    # BASELINE config 5's slicing: BFP16 x INT4, 64-row reads, 2-bit digits.
    "bfp16_int4": (WIDE["bfp16_int4"][0], WIDE["bfp16_int4"][1], 70, 300, 150),
    # 4-bit input digits (byte conversion path), 32-row reads, S-curve ADC.
    "int12_s4": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 3, 4, 4),
                      weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                      adc_bits=8), dict(write_variation=0.02, adc_nonlinearity=0.05), 45, 200, 70),
    # BFP8 inputs, stuck-at faults and shared read noise, a ragged vector block.
    "bfp8_p64": (dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                      weight_slice=(1, 1, 2, 2, 2), bw_e=4, array_size=(128, 64),
                      rows_per_read=64, adc_bits=(6, 7, 7, 8, 8)),
                 dict(write_variation=0.03, read_variation=0.02, stuck_at_low=0.01,
                      stuck_at_high=0.01), 130, 400, 100),
    # Four 2-bit weight slices at 64-row reads (32 KiB of terms per read: the middle
    # LDS capacity), 4-bit input digits.
    "int10_w4": (dict(activation_bits=10, weight_bits=7, input_slice=(1, 1, 4, 4),
                      weight_slice=(1, 2, 2, 2), array_size=(128, 64), rows_per_read=64,
                      adc_bits=8), dict(write_variation=0.02, drift_coefficient=0.05,
                                        drift_time=100.0), 90, 300, 130),
    # Voltage variation: real input operands (hi + lo of digit * (1 + vv*z)) instead of
    # digits; BFP16 x INT4 at 64-row reads with read noise and drift, and 4-bit digits at
    # 32-row reads with the S-curve ADC.
    "bfp16_voltage": (WIDE["bfp16_int4"][0],
                      dict(write_variation=0.02, read_variation=0.01, voltage_variation=0.03,
                           drift_coefficient=0.05, drift_time=100.0), 70, 300, 150),
    "int12_voltage": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 3, 4, 4),
                           weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                           adc_bits=8),
                      dict(write_variation=0.02, voltage_variation=0.05, adc_nonlinearity=0.05),
                      45, 200, 70),
    # slice_pair read noise: one plane of conductance terms per (weight, input) slice pair,
    # read from global memory; BFP16 x INT4 (nine input planes) with drift, and 4-bit digits
    # at 32-row reads with voltage variation and the S-curve ADC.
    "bfp16_slice_pair": (WIDE["bfp16_int4"][0],
                         dict(write_variation=0.02, read_variation=0.02, read_mode="slice_pair",
                              drift_coefficient=0.05, drift_time=100.0), 70, 300, 150),
    "int12_slice_pair_voltage": (dict(activation_bits=12, weight_bits=8, input_slice=(1, 3, 4, 4),
                                      weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32),
                                      rows_per_read=32, adc_bits=8),
                                 dict(write_variation=0.02, read_variation=0.01,
                                      read_mode="slice_pair", voltage_variation=0.03,
                                      adc_nonlinearity=0.05), 45, 200, 70),
}


def wide_mfma_case(name, seed):
    kwargs, effects, n, k, o = WIDE_MFMA[name]
    cfg = Config(**kwargs, nonidealities=Nonidealities(**effects))
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(n, k, generator=gen)
    a[:, ::17] *= 20     # outlier channels
    b = torch.randn(k, o, generator=gen) * 0.02
    return cfg, a, b


def flip_budget(cfg, diff):
    codes = diff.numel() * len(cfg.input_layout) * len(cfg.weight_layout)
    return max(1, 1e-4 * codes)


@pytest.mark.parametrize("name", list(WIDE_MFMA))
def test_wide_mfma_totals_with_injected_conductances(hip_device, name):
    """Same integer slice totals as the oracle given the same conductances, except ADC flips."""
    say("wide mfma totals", name)
    cfg, a, b = wide_mfma_case(name, 41)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    n, m, r = q.shape
    p = packed.shape[1]
    assert hip.mm_kernel(cfg, n, m, p) == 3
    seed, event = 777, 5
    raw, _, _ = oracle.restored(packed, cfg, seed, event, 0, p)
    expected = oracle.partial(q, packed, cfg, seed, event, 0, p, conductance=raw)
    got = hip.mm_totals_wide(q.to(hip_device), packed.to(hip_device), cfg, seed, event,
                             conductance=raw.to(hip_device)).cpu()
    assert got.dtype == torch.float64 and got.shape == expected.shape
    diff = got - expected.double()
    flips = int((diff != 0).sum())
    largest = max(abs(fa * fw) for _, _, fa in cfg.input_layout for _, _, fw in cfg.weight_layout)
    say("  totals differing", flips, "of", diff.numel(), "max", diff.abs().max().item())
    assert flips <= flip_budget(cfg, diff)
    assert diff.abs().max().item() <= 2 * largest


def test_wide_mfma_reference_vectors(hip_device, reference_vectors):
    """The reference's own totals for the BFP16 x INT4 case, given its conductances."""
    v = reference_vectors
    cfg = wide_case("bfp16_int4")
    q = torch.from_numpy(v["case_bfp16_int4_q"]).to(hip_device)
    packed = torch.from_numpy(v["case_bfp16_int4_packed"]).to(hip_device)
    seed = int(v["case_bfp16_int4_seed"])
    n, m, _ = q.shape
    assert hip.mm_kernel(cfg, n, m, packed.shape[1]) == 3
    raw = torch.from_numpy(v["case_bfp16_int4_restored"]).to(hip_device)
    got = hip.mm_totals_wide(q, packed, cfg, seed, 0, conductance=raw).cpu()
    expected = torch.from_numpy(v["case_bfp16_int4_totals"])
    diff = got - expected
    say("  reference totals differing", int((diff != 0).sum()), "of", diff.numel())
    assert int((diff != 0).sum()) <= flip_budget(cfg, diff)


@pytest.mark.parametrize("name", list(WIDE_MFMA))
def test_wide_mfma_sampled_conductances(hip_device, name):
    """Conductances sampled on the GPU (counter RNG, OCML) against the oracle's samples."""
    cfg, a, b = wide_mfma_case(name, 42)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    p = packed.shape[1]
    seed, event = 31337, 2
    expected = oracle.partial(q, packed, cfg, seed, event, 0, p)
    got = hip.mm_totals_wide(q.to(hip_device), packed.to(hip_device), cfg, seed, event).cpu()
    diff = got - expected.double()
    flips = int((diff != 0).sum())
    say("  sampled totals differing", flips, "of", diff.numel())
    assert flips <= flip_budget(cfg, diff)


@pytest.mark.parametrize("name", list(WIDE_MFMA))
def test_wide_mfma_epilogue_and_mm(hip_device, name):
    """Fused FP64 output = restore_scales + torch's FP64 read sum of the kernel's own totals,
    bit for bit; Simulator.mm within the flip budget of the oracle for two read events."""
    from memfast_amd import Simulator

    cfg, a, b = wide_mfma_case(name, 43)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    seed, event = 2024, 1
    totals = hip.mm_totals_wide(q.to(hip_device), packed.to(hip_device), cfg, seed, event).cpu()
    fused = hip.mm(q.to(hip_device), xs.to(hip_device), packed.to(hip_device), None,
                   ws.reshape(-1, p * c).to(hip_device), cfg, seed, event).cpu()
    assert fused.dtype == torch.float64
    restored = oracle.execute(q, xs, packed, ws, cfg, seed, event, p * c, totals=totals)
    assert bits_equal(fused, restored)
    sim = Simulator(cfg, device=hip_device)
    ad, bd = a.to(hip_device), b.to(hip_device)
    for ev in (0, 1):
        got = sim.mm(ad, bd)
        check_product(cfg, got, a, b, hip_device, event=ev, label=f"wide mfma {name} event {ev}")


def test_wide_mfma_column_chunks(hip_device):
    """A workspace of one 64-column chunk gives the same totals as the full workspace."""
    cfg, a, b = wide_mfma_case("bfp8_p64", 44)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    qd, pd = q.to(hip_device), packed.to(hip_device)
    full = hip.mm_totals_wide(qd, pd, cfg, 5, 0)
    n, m, r = q.shape
    p = packed.shape[1]
    import ctypes as ct

    lib = hip.library()
    per_block = len(cfg.weight_layout) * 32 * m * r * 3 * 2
    codes = (n * m * r * 2 + 255) // 256 * 256
    workspace = torch.empty(codes + 2 * per_block, dtype=torch.uint8, device=hip_device)
    chunked = torch.empty_like(full)
    q32, p32 = hip._u32(qd), hip._u32(pd)
    hip.check(lib.mf_mm_totals_wide(ct.byref(hip.descriptor(cfg)), hip._ptr(q32), n, m,
                                    hip._ptr(p32), p, None, 5, 0, hip._ptr(chunked),
                                    hip._ptr(workspace), workspace.numel(),
                                    hip._stream(qd.device)), "chunked totals")
    assert bits_equal(chunked, full)


# Groups align with the 64-row reads; 192, 320 and 1088 straddle the kernels'
# 256-row and 1024-column chunks; (64, 3) and (2, 64) take the 2-D group path.
WIDE_GROUPS = [((None, 1), (1, None)), ((64, 1), (1, 64)), ((192, 1), (1, 192)),
               ((320, 1), (1, 1088)), ((64, 3), (2, 64))]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("wgran,igran", WIDE_GROUPS, ids=[f"{w}-{i}" for w, i in WIDE_GROUPS])
def test_wide_group_quantizers_bit_exact(hip_device, wgran, igran, dtype):
    """FP64 group maxima (column, row and 2-D groups, chunk-straddling groups) -> codes and
    scales identical to the oracle's, from FP64 operands and from FP32 ones (widened inside
    the quantizers; 72 weight columns take the 16-byte loads of the column-group path)."""
    cfg = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                 weight_slice=(1, 1, 2), bw_e=8, array_size=(64, 64), adc_bits=(6, 6, 7),
                 weight_quant_gran=wgran, input_quant_gran=igran)
    gen = torch.Generator().manual_seed(45)
    a = torch.randn(9, 1500, generator=gen).to(dtype)
    a[:, 700] = 50.0
    b = (torch.randn(1500, 72, generator=gen) * 0.02).to(dtype)
    b[513, :] = -3.0
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, _, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    assert bits_equal(q.cpu().to(torch.int64) & 0xFFFF, q_ref & 0xFFFF)
    assert bits_equal(xs, xs_ref)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)


# Wide configurations with an INT operand of at most 8 bits: the reference quantizes each
# operand in its own dtype (FP32 up to 8 bits without BFP), so that operand's scales and
# codes are FP32 results even though the configuration restores in FP64.
MIXED_WIDTHS = [dict(activation_bits=16, weight_bits=4, weight_slice=(1, 1, 2)),
                dict(activation_bits=12, weight_bits=6),
                dict(activation_bits=8, weight_bits=12, input_slice=(1, 1, 2, 2, 2))]


@pytest.mark.parametrize("widths", MIXED_WIDTHS, ids=["a16w4", "a12w6", "a8w12"])
def test_mixed_width_operands_quantize_in_their_own_dtype(hip_device, widths):
    from memfast_amd import Simulator

    cfg = Config(**widths, array_size=(64, 32), rows_per_read=32, adc_bits=6,
                 weight_quant_gran=(32, 1), input_quant_gran=(1, 32),
                 nonidealities=Nonidealities(write_variation=0.0))
    assert cfg.wide
    gen = torch.Generator().manual_seed(46)
    a = torch.randn(24, 200, generator=gen)
    b = torch.randn(200, 70, generator=gen)
    # 8-bit inputs: quotients on and next to half-integers of their group's FP32 scale
    # (without the groups of huge peaks, whose products overflow FP32).
    groups = near_half_integer_groups(24, 7)
    groups[3::4] = groups[1::4]
    a[:, :32] = groups
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, _, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    mask = (1 << cfg.activation_bits) - 1
    assert bits_equal(q.cpu().to(torch.int64) & mask, q_ref & mask)
    assert bits_equal(xs, xs_ref)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)
    got = Simulator(cfg, device=hip_device).mm(a.to(hip_device), b.to(hip_device))
    assert bits_equal(got, oracle.mm(a, b, cfg))


# Narrow (FP32) group quantizers: whole-column and whole-matrix groups, groups that straddle
# the kernels' 256-row chunks, and 2-D groups (the row-first reduction path).
NARROW_GROUPS = [((None, 1), (1, None)), ((192, 1), (None, 64)), ((320, 3), (None, None)),
                 ((64, 70), (2, 64)), ((None, 7), (5, 128)), ((128, 2), (300, 1088))]


@pytest.mark.parametrize("wgran,igran", NARROW_GROUPS, ids=[f"{w}-{i}" for w, i in NARROW_GROUPS])
def test_narrow_group_quantizers_bit_exact(hip_device, wgran, igran):
    """FP32 group maxima of every group shape -> codes and scales identical to the oracle's."""
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(64, 64), adc_bits=8,
                 weight_quant_gran=wgran, input_quant_gran=igran)
    gen = torch.Generator().manual_seed(46)
    a = torch.randn(600, 1500, generator=gen)
    a[:, 700] = 50.0
    a[333, 10] = -80.0
    b = torch.randn(1500, 70, generator=gen) * 0.02
    b[513, :] = -3.0
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, _, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    assert bits_equal(q, q_ref) and bits_equal(xs, xs_ref)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)


@pytest.mark.parametrize("wgran", [(None, 1), (384, 1), (1024, 1)])
def test_tall_weight_groups_on_array_tiles_bit_exact(hip_device, wgran):
    """Tall column groups on 128x128 arrays (group maxima first, then the LDS code tile
    with each row's group scale) -> packed codes and scales identical to the oracle's."""
    say("tall weight groups", wgran)
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
                 adc_bits=8, weight_quant_gran=wgran, input_quant_gran=(1, 32))
    gen = torch.Generator().manual_seed(47)
    b = torch.randn(1500, 200, generator=gen) * 0.02
    b[700, 3] = 5.0
    b[1499, :] = -1.0
    packed, codes_t, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)
    assert bits_equal(codes_t, packed_columns(packed_ref))


def test_groups_of_one_read_share_the_scale_tables(hip_device):
    """Input groups (1, P) and weight groups (P, 1) with no padded reads or columns: the group
    grids are written straight into xscale and wscale (no gather) -> identical to the oracle."""
    say("groups of one read")
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                 adc_bits=8, weight_quant_gran=(32, 1), input_quant_gran=(1, 32))
    gen = torch.Generator().manual_seed(48)
    a = torch.randn(40, 256, generator=gen)
    a[7, 100] = 30.0
    b = torch.randn(256, 96, generator=gen)
    b[33, 5] = -9.0
    q, xs = hip.input_tiles(a.to(hip_device), cfg)
    packed, codes_t, ws = hip.weight_tiles(b.T.to(hip_device), cfg)
    q_ref, xs_ref = oracle.input_tiles(a, cfg)
    packed_ref, ws_ref = oracle.weight_tiles(b.T, cfg)
    assert bits_equal(q, q_ref) and bits_equal(xs, xs_ref)
    assert bits_equal(packed, packed_ref) and bits_equal(ws, ws_ref)
    assert bits_equal(codes_t, packed_columns(packed_ref))


def test_scale_aliasing_outside_groups_of_one_read_is_rejected(hip_device):
    """The C-ABI accepts scale == xscale / wscale only where the grid is the per-read table."""
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(64, 32), rows_per_read=32,
                 adc_bits=8, weight_quant_gran=(32, 1), input_quant_gran=(1, 32))
    descr = ct.byref(hip.descriptor(cfg))
    lib = hip.library()
    x = torch.zeros(4, 200, device=hip_device)   # k = 200: padded reads
    q = torch.empty(4, 256, dtype=torch.uint8, device=hip_device)
    xs = torch.empty(4, 8, device=hip_device)
    work = torch.empty(64, dtype=torch.int32, device=hip_device)
    rc = lib.mf_quantize_inputs(descr, hip._ptr(x), 4, 200, 200, 1, 32, hip._ptr(work),
                                hip._ptr(xs), hip._ptr(q), hip._ptr(xs), None,
                                hip._stream(hip_device))
    assert rc == hip.E_INVALID and b"alias" in lib.mf_last_error()
    w = torch.zeros(256, 90, device=hip_device)  # o = 90: padded columns
    packed = torch.empty(4, 3, 64, 32, dtype=torch.uint8, device=hip_device)
    ws = torch.empty(8, 96, device=hip_device)
    rc = lib.mf_quantize_weights(descr, hip._ptr(w), 256, 90, 90, 32, 1, hip._ptr(work),
                                 hip._ptr(ws), hip._ptr(packed), None, hip._ptr(ws), None,
                                 hip._stream(hip_device))
    assert rc == hip.E_INVALID and b"alias" in lib.mf_last_error()


def test_noisy_mfma_unsplit_epilogue(hip_device):
    """A grid of 512 blocks or more keeps the fused single-kernel read (no read split):
    its output is the reference epilogue of the kernel's own totals, bit for bit."""
    cfg = noisy_case("write")
    gen = torch.Generator().manual_seed(34)
    a = torch.randn(1024, 128, generator=gen)
    b = torch.randn(128, 2048, generator=gen)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    assert (p * c + 63) // 64 * ((n + 63) // 64) >= 512
    codes_t = packed_columns(packed).to(hip_device)
    totals = hip.mm_totals(q.to(hip_device), codes_t, cfg, 77, 2).cpu()
    fused = hip.mm(q.to(hip_device), xs.to(hip_device), packed.to(hip_device), codes_t,
                   ws.reshape(-1, p * c).to(hip_device), cfg, 77, 2).cpu()
    restored = oracle.execute(q, xs, packed, ws, cfg, 77, 2, p * c, totals=totals)
    assert bits_equal(fused, restored)


def test_noisy_terms_reused_across_reads(hip_device):
    """Write noise is event-independent: a programmed matrix samples its conductances
    once; later reads reuse them and give the same output as a fresh program, and
    reprogramming samples new ones."""
    from memfast_amd import AnalogMatrix, Simulator

    cfg = noisy_case("write")
    gen = torch.Generator().manual_seed(35)
    w = torch.randn(100, 200, generator=gen)
    x = torch.randn(40, 200, generator=gen).to(hip_device)
    sim = Simulator(cfg, device=hip_device)
    matrix = AnalogMatrix(w.to(hip_device), sim, name="layer")
    assert hip.mm_kernel(cfg, 40, 4, matrix.p) == 2
    first = matrix(x)
    assert matrix._terms_source is not None
    second = matrix(x)
    fresh = AnalogMatrix(w.to(hip_device), Simulator(cfg, device=hip_device), name="layer")(x)
    assert bits_equal(first, second) and bits_equal(second, fresh)
    check_product(cfg, second, x, w.T, hip_device, name="layer", event=1, label="reused terms")
    w2 = torch.randn(100, 200, generator=gen)
    matrix.update_weight(w2.T.to(hip_device))
    after = matrix(x)
    fresh2 = AnalogMatrix(w2.to(hip_device), Simulator(cfg, device=hip_device), name="layer")(x)
    assert bits_equal(after, fresh2)


def test_layer_input_and_bias_checks_in_one_status_read(hip_device):
    """AnalogLinear defers the finiteness check of its input to the read's status word:
    the reference's messages (memfast/quantization.py:12-13 grouped, :124-125 fixed scale),
    raised before the read event advances; a bias that overflows FP32 takes the FP64
    retry and then raises like the reference (simulator.py:612-615, :643-644)."""
    from torch import nn

    from memfast_amd import Simulator
    from memfast_amd.nn import AnalogLinear

    cfg = ideal(**CONFIG2 | dict(array_size=(64, 32), adc_bits=8, input_quant_gran=(1, 32)))
    torch.manual_seed(9)
    source = nn.Linear(70, 40)
    layer = AnalogLinear(source, Simulator(cfg, device=hip_device)).to(hip_device)
    x = torch.randn(5, 70, device=hip_device)
    good = layer(x)
    assert layer._event == 1
    bad = x.clone()
    bad[2, 3] = float("nan")
    with pytest.raises(ValueError, match="finite in torch.float32"):
        layer(bad)
    assert layer._event == 1
    layer.set_input_scale(0.05)
    with pytest.raises(ValueError, match=r"^quantized values must be finite$"):
        layer(bad)
    assert layer._event == 1
    layer.set_input_scale(None)
    again = layer(x)
    assert layer._event == 2 and bits_equal(again, good)
    # Output + bias beyond FP32 (FLT_MAX + ~1e32): the FP64 retry holds it, the cast back
    # to FP32 does not.
    layer.bias.fill_(torch.finfo(torch.float32).max)
    big = torch.full((2, 70), 1e32, device=hip_device)
    with pytest.raises(FloatingPointError):
        layer(big)
    assert layer._event == 2


def test_bounded_fixed_scale_reads_publish_their_input_check(hip_device, monkeypatch):
    """With fixed input scales whose restore cannot leave FP32 (every read's slice total
    is at most Config.reconstruction_bound), a layer read publishes its quantizer's status
    bits before the read and returns on them: the outputs equal the full status read's bit
    for bit (linear and convolution, FP32 and bfloat16 inputs); a non-finite input still
    raises before the event advances; an in-place bias change or a huge scale turns the
    bound off."""
    from torch import nn

    from memfast_amd import Simulator
    from memfast_amd.nn import AnalogConv2d, AnalogLinear
    from memfast_amd.simulator import AnalogMatrix

    cfg = noisy_case("write")
    torch.manual_seed(47)
    linear = nn.Linear(300, 90).to(hip_device)
    conv = nn.Conv2d(8, 16, 3, padding=1).to(hip_device)
    x = torch.randn(33, 300, device=hip_device)
    image = torch.randn(2, 8, 12, 12, device=hip_device)

    def build(source, kind):
        layer = kind(source, Simulator(cfg, device=hip_device), name="bounded")
        for matrix in getattr(layer, "matrices", [layer]):
            matrix.set_input_scale(0.03)
        return layer

    def read(source, kind, value, bounded):
        layer = build(source, kind)
        matrix = getattr(layer, "matrices", [layer])[0]
        seen = []
        original = AnalogMatrix._output_bounded

        def spy(self, arrays):
            seen.append(original(self, arrays) if bounded else False)
            return seen[-1]

        monkeypatch.setattr(AnalogMatrix, "_output_bounded", spy)
        with torch.no_grad():
            out = layer(value)
        monkeypatch.setattr(AnalogMatrix, "_output_bounded", original)
        assert seen and all(s == bounded for s in seen) and matrix._event == 1
        return out, layer

    for source, kind, value in ((linear, AnalogLinear, x), (conv, AnalogConv2d, image),
                                (linear, AnalogLinear, x.to(torch.bfloat16))):
        early, _ = read(source, kind, value, True)
        full, _ = read(source, kind, value, False)
        # bfloat16 widens to float32 exactly, so the float32 bits compare the bfloat16 bits.
        assert early.dtype == value.dtype and bits_equal(early.float(), full.float())

    # float16 outputs keep the host scan of the cast: a bounded FP32 output past float16's
    # range still raises.
    layer = build(linear, AnalogLinear)
    with torch.no_grad():
        layer.bias.fill_(1e5)
    assert layer._output_bounded(-(-300 // cfg.array_size[0]))
    with pytest.raises(FloatingPointError):
        layer(x.half())
    assert layer._event == 0

    layer = build(linear, AnalogLinear)
    bad = x.clone()
    bad[4, 7] = float("inf")
    assert layer._output_bounded(-(-300 // cfg.array_size[0]))
    with pytest.raises(ValueError, match=r"^quantized values must be finite$"):
        layer(bad)
    assert layer._event == 0
    with torch.no_grad():
        layer.bias.fill_(torch.finfo(torch.float32).max)
    assert not layer._output_bounded(-(-300 // cfg.array_size[0]))
    layer.set_input_scale(1e37)
    with torch.no_grad():
        layer.bias.zero_()
    assert not layer._output_bounded(-(-300 // cfg.array_size[0]))
    assert torch.isfinite(layer(x[:3])).all() and layer._event == 1


EXTENT_CASES = [
    ("ideal", ideal(**CONFIG2 | dict(array_size=(64, 32))), 9, 200, 70),
    ("ideal_258_reads", ideal(**CONFIG2 | dict(array_size=(64, 32))), 3, 8200, 40),
    ("write_split", noisy_case("write"), 9, 200, 70),
    ("shared_unsplit", noisy_case("rows64"), 1030, 300, 2040),
]


@pytest.mark.parametrize("name,cfg,n,k,o", EXTENT_CASES, ids=[c[0] for c in EXTENT_CASES])
def test_logical_extent_matches_full_read(hip_device, name, cfg, n, k, o):
    """Computing only the logical output columns and skipping reads wholly in the zero
    padding past row K gives the same outputs, bit for bit, as the full read."""
    gen = torch.Generator().manual_seed(46)
    a = torch.randn(n, k, generator=gen).to(hip_device)
    b = torch.randn(k, o, generator=gen).to(hip_device)
    q, xs = hip.input_tiles(a, cfg)
    packed, packed_t, ws = hip.weight_tiles(b.T, cfg)
    nq, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    kernel = hip.mm_kernel(cfg, nq, m, p)
    assert kernel in (1, 2)
    assert m * cfg.reads_per_array > -(-k // cfg.read_rows)     # some reads are all padding
    full = hip.mm(q, xs, packed, packed_t, ws.reshape(-1, p * c), cfg, 11, 4)
    part = hip.mm(q, xs, packed, packed_t, ws.reshape(-1, p * c), cfg, 11, 4, out_cols=o,
                  k_rows=k)
    assert bits_equal(part[:, :o], full[:, :o])
