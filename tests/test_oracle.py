"""Pins of the CPU oracle (oracle/oracle.py) against reference-held data and mathematics.

* LeNet checkpoints shipped with the reference: INT4 codes, packing, seeds.
* The DFT notebook known answer (examples/notebooks/03_dft_image_denoising.ipynb:374-386).
* Vectors written by tests/golden/make_reference_vectors.py from the reference CPU path.
* A scalar C restatement (oracle/brute.c) of the ideal ADC closed form and the RNG hash.
"""

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import fixture_config
from memfast_amd import Config, Nonidealities
from oracle import oracle

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


@pytest.fixture(scope="module")
def brute():
    lib_path = ROOT / "oracle" / "libbrute.so"
    if not lib_path.exists():
        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    lib = ctypes.CDLL(str(lib_path))
    lib.brute_mix.argtypes = [ctypes.c_uint32]
    lib.brute_mix.restype = ctypes.c_uint32
    lib.brute_uniform_bits.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32]
    lib.brute_uniform_bits.restype = ctypes.c_uint32
    lib.brute_event_seed.argtypes = [ctypes.c_uint32, ctypes.c_uint64]
    lib.brute_event_seed.restype = ctypes.c_uint64
    return lib


def _cfg(case, **extra):
    base = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                weight_quant_gran=(16, 1), input_quant_gran=(1, 16), adc_bits=(6, 7, 7, 8, 8))
    noise = {
        "ideal": dict(write_variation=0.0),
        "write": dict(write_variation=0.02),
        "shared": dict(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1),
        "slice_pair": dict(write_variation=0.02, read_variation=0.02, read_mode="slice_pair"),
        "output": dict(write_variation=0.02, read_variation=0.02, read_mode="output"),
        "voltage": dict(write_variation=0.0, voltage_variation=0.05),
        "saf_drift": dict(write_variation=0.02, stuck_at_low=0.05, stuck_at_high=0.03,
                          drift_coefficient=0.05, drift_time=100.0),
        "binary_int4": dict(write_variation=0.02),
        "bfp16_int4": dict(write_variation=0.02, read_variation=0.01, drift_coefficient=0.05,
                           drift_time=100.0),
        "int12_ideal": dict(write_variation=0.0),
        "bfp8_binary": dict(write_variation=0.02, adc_nonlinearity=0.05),
    }[case]
    if case in WIDE_CASES:
        base = dict(WIDE_CASES[case])
    elif case == "binary_int4":
        base = dict(activation_bits=8, weight_bits=4, array_size=(64, 64), adc_bits=6)
    base.update(extra)
    return Config(**base, nonidealities=Nonidealities(**noise))


# Wide configurations of the fixture (precision above 8 bits or BFP).
WIDE_CASES = {
    "bfp16_int4": dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                       weight_slice=(1, 1, 2), bw_e=8, array_size=(64, 64), adc_bits=(6, 6, 7)),
    "int12_ideal": dict(activation_bits=12, weight_bits=10, array_size=(32, 16), rows_per_read=16,
                        adc_bits=8),
    "bfp8_binary": dict(activation_bits=8, weight_bits=8, bw_e=4, array_size=(32, 16),
                        rows_per_read=16, adc_bits=6),
}


def test_bfp_exponents_at_power_of_two_edges(reference_vectors):
    """BFP scales/codes around 2^k (floor(log2(max)), quantization.py:35-40)."""
    v = reference_vectors
    edges = torch.from_numpy(v["bfp_edges_in"])
    for bits, bw_e in ((16, 8), (12, 5), (8, 11)):
        code, scale = oracle.grouped_quantize(edges, bits, (1, 4), bw_e)
        np.testing.assert_array_equal(code.numpy(), v[f"bfp_edges_code_{bits}_{bw_e}"])
        np.testing.assert_array_equal(scale.numpy(), v[f"bfp_edges_scale_{bits}_{bw_e}"])


# ---------------------------------------------------------------------------
# RNG
# ---------------------------------------------------------------------------
def test_rng_matches_reference_vectors(reference_vectors):
    v = reference_vectors
    addresses = torch.from_numpy(v["rng_address"])
    for si, seed in enumerate(v["rng_seeds"].tolist()):
        for ti, stream in enumerate(v["rng_streams"].tolist()):
            u = oracle.uniform(addresses, int(seed), int(stream)).numpy()
            z = oracle.normal(addresses, int(seed), int(stream)).numpy()
            np.testing.assert_array_equal(u, v["rng_uniform"][si, ti])
            np.testing.assert_array_equal(z, v["rng_normal"][si, ti])


def test_event_seed_and_mix_vectors(reference_vectors, brute):
    v = reference_vectors
    for (seed, event), expected in zip(v["event_pairs"].tolist(), v["event_seeds"].tolist()):
        assert oracle.event_seed(int(seed), int(event)) == expected
        assert brute.brute_event_seed(int(seed), int(event)) == expected
    for x, expected in zip(v["mix_in"].tolist(), v["mix_out"].tolist()):
        assert oracle.mix_int(int(x)) == expected
        assert brute.brute_mix(int(x)) == expected


def test_uniform_c_restatement(reference_vectors, brute):
    v = reference_vectors
    for si, seed in enumerate(v["rng_seeds"].tolist()):
        for ti, stream in enumerate(v["rng_streams"].tolist()):
            bits = np.array([brute.brute_uniform_bits(int(a) & (2**64 - 1), int(seed), int(stream))
                             for a in v["rng_address"].tolist()], dtype=np.float64)
            np.testing.assert_array_equal(((bits + 0.5) / 2**24).astype(np.float32),
                                          v["rng_uniform"][si, ti])


def test_uniform_distribution():
    """Uniforms are FP32(h + 0.5) / 2^24 for 24-bit h: multiples of 2^-25 in (0,1)."""
    address = torch.arange(200000, dtype=torch.int64) * 7919 + 2**33
    u = oracle.uniform(address, 4017293833, 10).double()
    scaled = u * 2**25
    assert torch.equal(scaled, scaled.round())
    assert 0 < u.min() and u.max() < 1
    assert abs(u.mean().item() - 0.5) < 3e-3
    counts = torch.histc(u, bins=16, min=0, max=1)
    expected = len(u) / 16
    chi2 = ((counts - expected) ** 2 / expected).sum().item()
    assert chi2 < 40  # 15 dof, p ~ 5e-4
    z = oracle.normal(address, 4017293833, 10).double()
    assert abs(z.mean().item()) < 0.01 and abs(z.std().item() - 1) < 0.01


def test_seed_names_from_checkpoint():
    data = np.load(GOLDEN / "lenet_int4.npz", allow_pickle=False)
    for index in range(int(data["count"])):
        name = str(data[f"l{index}_name"])
        assert oracle.name_seed(135, name) == int(data[f"l{index}_seed"])
    assert oracle.name_seed(135, "matrix.0") == 4017293833
    assert oracle.name_seed(135, "matrix.1") == 3292730091


# ---------------------------------------------------------------------------
# Quantization / packing
# ---------------------------------------------------------------------------
def test_lenet_int4_codes_from_float_checkpoint():
    data = np.load(GOLDEN / "lenet_int4.npz", allow_pickle=False)
    cfg = Config(activation_bits=8, weight_bits=4, array_size=(64, 64), adc_bits=6,
                 input_quant_gran=(1, None), weight_quant_gran=(None, 1))
    for index in range(int(data["count"])):
        weight = torch.from_numpy(data[f"l{index}_weight"])
        packed, scale = oracle.weight_tiles(weight, cfg)
        np.testing.assert_array_equal(packed.numpy(), data[f"l{index}_packed"])
        stored = torch.from_numpy(data[f"l{index}_weight_scale"])
        # The shipped scales came from a CUDA reciprocal multiply; the CPU reference
        # divides.  They agree to 1 ulp.
        ulp = torch.nextafter(stored, torch.full_like(stored, math.inf)) - stored
        assert ((scale - stored).abs() <= ulp).all()
        peak = weight.abs().amax(1)
        expected = torch.where(peak > 0, peak, torch.ones_like(peak)) / 7
        o = weight.shape[0]
        assert torch.equal(scale.reshape(scale.shape[0], -1)[0, :o], expected)


def test_fixed_input_scale_fixture():
    data = np.load(GOLDEN / "lenet_int4.npz", allow_pickle=False)
    for index in range(int(data["count"])):
        maximum = float(data[f"l{index}_maximum"])
        scale = max(maximum if maximum > 0 else 1.0, torch.finfo(torch.float32).tiny) / 127
        stored = data[f"l{index}_input_scale"]
        assert np.all(stored == np.float32(scale))


def test_round_half_even_and_clamp():
    cfg = Config(activation_bits=4, weight_bits=4, array_size=(8, 4), input_quant_gran=(1, None))
    # max 7 -> scale 1; values at .5 boundaries round to even.
    x = torch.tensor([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, -7.0]])
    q, xs = oracle.input_tiles(x, cfg)
    codes = q.flatten().long()
    signed = torch.where(codes >= 8, codes - 16, codes)
    assert signed.tolist() == [7, 0, 2, 2, 0, -2, -2, -7]
    assert xs.flatten().tolist() == [1.0]


def test_read_starts_and_padding():
    cfg = Config(array_size=(10, 4), rows_per_read=4, input_quant_gran=(1, None),
                 weight_quant_gran=(None, 1))
    assert oracle.read_starts(2, cfg).tolist() == [0, 4, 8, 10, 14, 18]
    x = torch.arange(1, 16, dtype=torch.float32)[None]  # K=15 -> m=2, padded to 20
    q, xs = oracle.input_tiles(x, cfg)
    assert q.shape == (1, 2, 10) and xs.shape == (1, 6)
    assert q.flatten()[15:].tolist() == [0] * 5


def test_reference_fixture_tiles(reference_vectors):
    v = reference_vectors
    for name in v["case_names"].tolist():
        cfg = fixture_config(v, name)
        a = torch.from_numpy(v[f"case_{name}_a"])
        b = torch.from_numpy(v[f"case_{name}_b"])
        packed, wscale = oracle.weight_tiles(b.T, cfg)
        q, xscale = oracle.input_tiles(a, cfg)
        np.testing.assert_array_equal(packed.numpy(), v[f"case_{name}_packed"])
        np.testing.assert_array_equal(wscale.numpy(), v[f"case_{name}_wscale"])
        np.testing.assert_array_equal(q.numpy(), v[f"case_{name}_q"])
        np.testing.assert_array_equal(xscale.numpy(), v[f"case_{name}_xscale"])


def test_fixture_configs_match_the_case_table(reference_vectors):
    """The configurations stored with the vectors are the ones this file's table names."""
    v = reference_vectors
    names = v["case_names"].tolist()
    for name in names:
        if not name.startswith("precise"):
            assert repr(fixture_config(v, name)) == repr(_cfg(name)), name
    precise = [name for name in names if name.startswith("precise")]
    assert len(precise) == 4
    for name in precise:
        cfg = fixture_config(v, name)
        assert cfg.precise_currents and oracle.precise_currents(cfg), name


# ---------------------------------------------------------------------------
# Array reads
# ---------------------------------------------------------------------------
def test_reference_fixture_reads(reference_vectors):
    v = reference_vectors
    for name in v["case_names"].tolist():
        cfg = fixture_config(v, name)
        packed = torch.from_numpy(v[f"case_{name}_packed"])
        q = torch.from_numpy(v[f"case_{name}_q"])
        seed = int(v[f"case_{name}_seed"])
        p = packed.shape[1]
        raw, _, _ = oracle.restored(packed, cfg, seed, 0, 0, p)
        np.testing.assert_array_equal(raw.numpy(), v[f"case_{name}_restored"])
        totals = oracle.partial(q, packed, cfg, seed, 0, 0, p)
        np.testing.assert_array_equal(totals.numpy(), v[f"case_{name}_totals"])


def test_reference_fixture_mm(reference_vectors):
    v = reference_vectors
    for name in v["case_names"].tolist():
        cfg = fixture_config(v, name)
        a = torch.from_numpy(v[f"case_{name}_a"])
        b = torch.from_numpy(v[f"case_{name}_b"])
        np.testing.assert_array_equal(oracle.mm(a, b, cfg).numpy(), v[f"case_{name}_out0"])
        np.testing.assert_array_equal(oracle.mm(a, b, cfg, event=1).numpy(),
                                      v[f"case_{name}_out1"])


def _brute_totals(brute, q, packed, cfg):
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    il, wl = oracle.input_layout(cfg), oracle.weight_layout(cfg)
    gr = oracle.reads_per_array(cfg)
    out = np.zeros((n, m * gr, p, c), dtype=np.int64)
    ints = lambda values: (ctypes.c_int * len(values))(*values)
    longs = lambda values: (ctypes.c_int64 * len(values))(*values)
    wide = q.dtype != torch.uint8
    dtype = np.int64 if wide else np.uint8
    qn = np.ascontiguousarray(q.numpy().astype(dtype))
    pn = np.ascontiguousarray(packed.numpy().astype(dtype))
    entry = brute.brute_ideal_totals_wide if wide else brute.brute_ideal_totals
    entry(
        qn.ctypes.data_as(ctypes.c_void_p), pn.ctypes.data_as(ctypes.c_void_p), n, m, p, r, c,
        oracle.read_rows(cfg), len(il), ints([e[0] for e in il]), longs([e[1] for e in il]),
        longs([e[2] for e in il]), len(wl), ints([e[0] for e in wl]), longs([e[1] for e in wl]),
        longs([e[2] for e in wl]), longs(oracle.adc_maxima(cfg)),
        out.ctypes.data_as(ctypes.c_void_p),
    )
    return out


@pytest.mark.parametrize("kwargs,shape", [
    (dict(array_size=(32, 16), rows_per_read=16, input_slice=(1, 1, 2, 2, 2),
          weight_slice=(1, 1, 2, 2, 2), adc_bits=(6, 7, 7, 8, 8)), (5, 70, 40)),
    (dict(array_size=(20, 8), rows_per_read=7, adc_bits=4), (3, 45, 9)),
    (dict(activation_bits=6, weight_bits=4, array_size=(16, 8), weight_slice=(1, 3), adc_bits=3),
     (4, 40, 11)),
    (dict(weight_bits=4, weight_signed=False, weight_slice=(2, 2), array_size=(16, 4),
          adc_bits=5), (2, 33, 6)),
])
def test_ideal_partial_matches_closed_form_and_brute(brute, kwargs, shape):
    cfg = Config(**kwargs, nonidealities=Nonidealities(write_variation=0.0))
    torch.manual_seed(7)
    n, k, o = shape
    a = torch.randn(n, k)
    b = torch.randn(k, o).abs() if not cfg.weight_signed else torch.randn(k, o)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    q, _ = oracle.input_tiles(a, cfg)
    totals = oracle.partial(q, packed, cfg, 1, 0, 0, packed.shape[1])
    closed = oracle.ideal_totals_closed_form(q, packed, cfg)
    assert torch.equal(totals.long(), closed)
    assert np.array_equal(_brute_totals(brute, q, packed, cfg), closed.numpy())


@pytest.mark.parametrize("name", ["precise_slice9_ideal", "precise_close_ideal"])
def test_precise_ideal_fixtures_match_closed_form_and_brute(brute, reference_vectors, name):
    """FP64 currents (a 9-bit slice; high - low < 1e-4 high) with ideal devices: the
    reference's totals, the oracle's and the C brute force of min(sum da*dw, max) agree."""
    v = reference_vectors
    cfg = fixture_config(v, name)
    q = torch.from_numpy(v[f"case_{name}_q"])
    packed = torch.from_numpy(v[f"case_{name}_packed"])
    reference = torch.from_numpy(v[f"case_{name}_totals"])
    closed = oracle.ideal_totals_closed_form(q, packed, cfg)
    assert torch.equal(reference.long(), closed) and torch.equal(reference, closed.to(reference.dtype))
    totals = oracle.partial(q, packed, cfg, int(v[f"case_{name}_seed"]), 0, 0, packed.shape[1])
    assert totals.dtype == reference.dtype and torch.equal(totals, reference)
    assert np.array_equal(_brute_totals(brute, q, packed, cfg), closed.numpy())
    # Clamping happens: the cases reach the ADC limits, so min() is exercised.
    assert int(closed.abs().max()) > 0


def test_dft_known_answer():
    """examples/notebooks/03_dft_image_denoising.ipynb:374-386 (recorded max error 9.537e-07)."""
    size = 256
    idx = np.arange(size)
    basis = np.exp(-2j * np.pi * np.outer(idx, idx) / size) / np.sqrt(size)
    weight = torch.tensor(basis.real, dtype=torch.float32)
    vectors = torch.linspace(-1, 1, 3 * size).reshape(3, size)
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1,) * 8, weight_slice=(1,) * 8,
                 array_size=(64, 64), adc_bits=8, input_quant_gran=(1, 64),
                 weight_quant_gran=(None, 1), seed=135,
                 nonidealities=Nonidealities(write_variation=0.0))
    wscale = weight.abs().amax(dim=0, keepdim=True) / 127
    groups = vectors.reshape(3, size // 64, 64)
    iscale = (groups.abs().amax(dim=-1, keepdim=True) / 127).expand_as(groups).reshape_as(vectors)
    dq_w = (weight / wscale).round().clamp(-127, 127) * wscale
    dq_x = (vectors / iscale).round().clamp(-127, 127) * iscale
    expected = dq_x @ dq_w
    actual = oracle.mm(vectors, weight, cfg)
    # The notebook's own assertion; its recorded 9.537e-07 came from the CUDA path,
    # whose summation order differs from the CPU reference's.
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=2e-5)


# ---------------------------------------------------------------------------
# Flip accounting (oracle/flips.py) and chunked execution, pinned by planted mistakes
# ---------------------------------------------------------------------------
def _flip_case():
    from oracle import flips  # noqa: F401

    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                 adc_bits=(6, 7, 7, 8, 8), nonidealities=Nonidealities(write_variation=0.02))
    gen = torch.Generator().manual_seed(61)
    a = torch.randn(6, 70, generator=gen)
    b = torch.randn(70, 40, generator=gen)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    totals = oracle.partial(q, packed, cfg, 5, 0, 0, packed.shape[1])
    out = oracle.execute(q, xs, packed, ws, cfg, 5, 0, 40, totals=totals)
    return cfg, q, xs, packed, ws, totals, out


def test_flip_accounting_accepts_one_planted_flip():
    """One code of pair (a=1, w=2) moved by one count: one flip, one flagged output, the
    output moved by exactly its effect, every other output unchanged."""
    from oracle import flips

    cfg, q, xs, packed, ws, totals, out = _flip_case()
    fa, fw = cfg.input_layout[1][2], cfg.weight_layout[2][2]
    moved = totals.clone()
    moved[2, 3, 1, 5] += fa * fw
    got = oracle.execute(q, xs, packed, ws, cfg, 5, 0, 40, totals=moved)
    report = flips.check_noisy(cfg, got, out, moved, totals, xscale=xs, wscale=ws)
    assert report["differing"] == 1 and report["flips"] == 1
    assert report["flagged_outputs"] == 1 and report["clean_inexact"] == 0
    assert got[2, 16 + 5] != out[2, 16 + 5]


def test_flip_accounting_counts_multiple_flips_in_one_total():
    from oracle import flips

    cfg, *_, totals, _ = _flip_case()
    factors = flips.pair_factors(cfg)
    moved = totals.clone()
    moved[0, 0, 0, 0] += factors[0] - factors[7] + factors[24]
    _, count, unexplained, _ = flips.count_flips(cfg, moved, totals)
    assert unexplained == 0 and count >= 2


def test_flip_accounting_rejects_planted_mistakes():
    """Planted in the oracle's own output: a difference no three single-count flips
    explain, an unflipped output off by 1e-4, a flipped output that moved too far, and
    more flips than the 1e-4 budget all fail."""
    from oracle import flips

    cfg, q, xs, packed, ws, totals, out = _flip_case()
    bad = totals.clone()
    bad[1, 1, 0, 1] += 7777
    with pytest.raises(AssertionError, match="beyond three code flips"):
        flips.check_noisy(cfg, out, out, bad, totals)
    wrong = out.clone()
    wrong[4, 7] *= 1 + 1e-4
    with pytest.raises(AssertionError, match="1e-5 relative"):
        flips.check_noisy(cfg, wrong, out, totals, totals)
    moved = totals.clone()
    moved[3, 2, 0, 9] += 1
    far = oracle.execute(q, xs, packed, ws, cfg, 5, 0, 40, totals=moved)
    far[3, 9] += 10 * abs(float(far[3, 9] - out[3, 9])) + 1e-3
    with pytest.raises(AssertionError, match="more than their flips explain"):
        flips.check_noisy(cfg, far, out, moved, totals, xscale=xs, wscale=ws)
    many = totals.clone()
    many[:, :, :, :] += 1
    with pytest.raises(AssertionError, match="budget"):
        flips.check_noisy(cfg, out, out, many, totals)


def test_execute_tiles_equals_full_columns():
    """oracle.execute(tiles=...) returns exactly the full product's columns of those tiles."""
    cfg = Config(activation_bits=8, weight_bits=8, array_size=(32, 16), rows_per_read=16,
                 adc_bits=8, nonidealities=Nonidealities(write_variation=0.02))
    gen = torch.Generator().manual_seed(62)
    a = torch.randn(5, 70, generator=gen)
    b = torch.randn(70, 90, generator=gen)
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.T, cfg)
    full = oracle.execute(q, xs, packed, ws, cfg, 9, 2, 96)
    for tiles in ((0, 2), (2, 4), (4, 6), (2, 3)):
        part = oracle.execute(q, xs, packed, ws, cfg, 9, 2, 96, tiles=tiles)
        assert torch.equal(part, full[:, tiles[0] * 16:tiles[1] * 16])
    with pytest.raises(ValueError):
        oracle.execute(q, xs, packed, ws, cfg, 9, 2, 96, tiles=(1, 3))


@pytest.mark.parametrize("wide", [False, True])
def test_zero_point_correction_closed_form(wide):
    """map_quantized with zero points (simulator.py:173-185, :587-611): with ideal devices
    and an ADC that never clamps (max 2^12-1 > 32 rows x 3 x 3 per pair), the read equals
    x_dequantized @ (scale * (code - zero_point)).T up to rounding; a dropped or
    sign-flipped correction misses by the zero points' whole contribution."""
    cfg = Config(activation_bits=12 if wide else 8, weight_bits=4, weight_signed=False,
                 input_slice=(1, 1, 2, 2, 2, 2, 2) if wide else (1, 1, 2, 2, 2),
                 weight_slice=(2, 2), array_size=(64, 32), rows_per_read=32, adc_bits=12,
                 input_quant_gran=(1, 32), nonidealities=Nonidealities(write_variation=0.0))
    gen = torch.Generator().manual_seed(63)
    o, k = 40, 150
    codes = torch.randint(0, 16, (o, k), generator=gen)
    scales = torch.rand(o, 1, generator=gen) * 0.1 + 0.01
    zero_points = torch.randint(3, 12, (o, 1), generator=gen).float()
    x = torch.randn(6, k, generator=gen, dtype=torch.float64 if wide else torch.float32)
    packed, wscale, correction = oracle.imported_tiles(codes, scales, cfg, zero_points)
    q, xs = oracle.input_tiles(x, cfg)
    got = oracle.execute(q, xs, packed, wscale, cfg, 1, 0, o, zero_correction=correction)
    bits = cfg.activation_bits
    signed = (q.long().reshape(6, -1)[:, :k] & ((1 << bits) - 1))
    signed = (signed ^ (1 << (bits - 1))) - (1 << (bits - 1))
    per_row_scale = xs.repeat_interleave(32, dim=1)[:, :k]
    dequantized = signed.double() * per_row_scale.double()
    expected = dequantized @ (scales.double() * (codes.double() - zero_points.double())).T
    torch.testing.assert_close(got.double(), expected, rtol=1e-5, atol=1e-5)
    without = oracle.execute(q, xs, packed, wscale, cfg, 1, 0, o)
    assert (without.double() - expected).abs().max() > 1e-2


def _boundary_case(**effects):
    cfg = Config(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                 weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                 adc_bits=(6, 7, 7, 9, 9), nonidealities=Nonidealities(**effects))
    gen = torch.Generator().manual_seed(62)
    a = torch.randn(12, 70, generator=gen)
    b = torch.randn(70, 40, generator=gen)
    q, _ = oracle.input_tiles(a, cfg)
    packed, _ = oracle.weight_tiles(b.T, cfg)
    raw, _, _ = oracle.restored(packed, cfg, 11, 2, 0, packed.shape[1])
    return cfg, q, packed, raw


@pytest.mark.parametrize("effects", [
    dict(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1),
    dict(write_variation=0.02, stuck_at_low=0.05, drift_coefficient=0.05, drift_time=100.0),
])
def test_exact_adc_arguments_round_to_the_oracle_codes(effects):
    """flips.adc_arguments restates the ADC argument (memfast/reference.py:54-60, 96-115)
    in exact arithmetic: rounding and clamping it gives the oracle's per-pair codes except
    within FP32 rounding distance of a boundary.  Leaving out the S-curve, the 1/unit
    scale or the low level moves hundreds of codes."""
    from oracle import flips

    cfg, q, packed, raw = _boundary_case(**effects)
    p = packed.shape[1]
    codes = {}
    oracle.partial(q, packed, cfg, 11, 2, 0, p, conductance=raw, codes=codes)
    y = flips.adc_arguments(q, packed, cfg, raw)
    maxima = torch.tensor(cfg.adc_maxima, dtype=torch.float64)[None, None, None, :, None]
    exact = torch.minimum(y.clamp(min=0), maxima).round()
    distance = (y - y.floor() - 0.5).abs() / y.abs().clamp(min=1.0)
    n, groups = q.shape[0], q.shape[1] * cfg.reads_per_array
    mismatched = far = 0
    for (ai, wi), count in codes.items():
        count = count.reshape(n, groups, -1).double()
        differs = count != exact[:, :, ai, wi]
        mismatched += int(differs.sum())
        far += int((differs & (distance[:, :, ai, wi] > 2.0**-18)).sum())
    assert far == 0 and mismatched <= 2
    # Planted mistakes in the restatement (no S-curve, another span or low level; the read
    # voltage cancels) are caught by the same comparison.
    for wrong in (dict(adc_nonlinearity=0.0), dict(high_conductance=1.1e-5),
                  dict(low_conductance=2e-7)):
        if "adc_nonlinearity" in wrong and not cfg.nonidealities.adc_nonlinearity:
            continue
        from dataclasses import replace

        bad = replace(cfg, nonidealities=replace(cfg.nonidealities, **wrong)) \
            if "adc_nonlinearity" in wrong else replace(cfg, **wrong)
        moved = (torch.minimum(flips.adc_arguments(q, packed, bad, raw).clamp(min=0),
                               maxima).round() != exact).sum()
        assert int(moved) > 100, wrong


def test_boundary_flips_accept_only_flips_at_rounding_boundaries():
    """A planted flip of the pair nearest its rounding boundary is explained; one of a
    pair far from every boundary is not."""
    from oracle import flips

    cfg, q, packed, raw = _boundary_case(write_variation=0.02, read_variation=0.01,
                                         adc_nonlinearity=0.1)
    p, c = packed.shape[1], cfg.array_size[1]
    totals = oracle.partial(q, packed, cfg, 11, 2, 0, p, conductance=raw)
    y = flips.adc_arguments(q, packed, cfg, raw)
    maxima = torch.tensor(cfg.adc_maxima, dtype=torch.float64)[None, None, None, :, None]
    inside = (y > 0) & (y < maxima)
    distance = torch.where(inside, (y - y.floor() - 0.5).abs(), torch.full_like(y, 9.0))
    n, groups = totals.shape[:2]
    factors = [[fa * fw for _, _, fw in cfg.weight_layout] for _, _, fa in cfg.input_layout]
    for pick, expect in ((distance.argmin(), True), ((distance - 0.25).abs().argmin(), False)):
        v, g, a, w, col = np.unravel_index(int(pick), tuple(distance.shape))
        moved = totals.clone().reshape(n, groups, -1)
        moved[v, g, col] += factors[a][w]
        differing, count, worst, unexplained = flips.boundary_flips(
            cfg, moved.reshape(totals.shape), totals, y, 2.0**-18)
        assert differing == 1
        if expect:
            assert count == 1 and not unexplained and worst <= 2.0**-18
        else:
            assert count == 0 and len(unexplained) == 1
