"""Config / Nonidealities: derived layouts and validation (memfast/config.py)."""

import itertools

import pytest

from memfast_amd import Config, Nonidealities
from oracle import oracle

BASELINE = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
                weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))


def test_baseline_layout_values():
    cfg = Config(**BASELINE)
    # LSB-first: widths (1,1,2,2,2) reversed -> 2,2,2,1,1; sign slice has factor -128.
    expected = ((0, 3, 1), (2, 3, 4), (4, 3, 16), (6, 1, 64), (7, 1, -128))
    assert cfg.input_layout == expected
    assert cfg.weight_layout == expected
    assert cfg.adc_maxima == (255, 255, 127, 127, 63)
    assert cfg.read_rows == 32 and cfg.reads_per_array == 4
    assert not cfg.wide and not cfg.precise_currents


@pytest.mark.parametrize("widths,bits", [((1,) * 8, 8), ((1, 3, 4), 8), ((1, 1, 2), 4),
                                          ((1, 7), 8), (None, 6)])
def test_layout_reconstructs_every_code(widths, bits):
    """Sum of factor*digit over the layout equals the two's complement value."""
    cfg = Config(activation_bits=bits, weight_bits=bits, input_slice=widths, weight_slice=widths)
    for code in range(-(1 << (bits - 1)), 1 << (bits - 1)):
        stored = code & ((1 << bits) - 1)
        value = sum(f * ((stored >> s) & m) for s, m, f in cfg.input_layout)
        assert value == code


def test_unsigned_layout_positive():
    cfg = Config(weight_bits=4, weight_signed=False, weight_slice=(2, 2))
    assert cfg.weight_layout == ((0, 3, 1), (2, 3, 4))
    for code in range(16):
        assert sum(f * ((code >> s) & m) for s, m, f in cfg.weight_layout) == code


@pytest.mark.parametrize("kwargs", [
    dict(BASELINE),
    dict(activation_bits=4, weight_bits=6, adc_bits=5, array_size=(48, 12), rows_per_read=7),
    dict(weight_slice=(1, 3, 4), adc_bits=(3, 5, 9), array_size=(64, 32)),
])
def test_derived_properties_match_oracle(kwargs):
    cfg = Config(**kwargs)
    assert cfg.input_layout == oracle.input_layout(cfg)
    assert cfg.weight_layout == oracle.weight_layout(cfg)
    assert cfg.adc_maxima == oracle.adc_maxima(cfg)
    assert cfg.read_rows == oracle.read_rows(cfg)
    assert cfg.reads_per_array == oracle.reads_per_array(cfg)
    assert cfg.precise_currents == oracle.precise_currents(cfg)
    assert cfg.wide == oracle.is_wide(cfg)


def test_adc_bits_msb_first():
    cfg = Config(weight_slice=(1, 1, 2, 2, 2), adc_bits=(6, 7, 8, 9, 10))
    assert cfg.adc_maxima == (1023, 511, 255, 127, 63)
    assert cfg.adc_maximum == 1023


def test_reads_ragged():
    cfg = Config(array_size=(100, 8), rows_per_read=30)
    assert cfg.reads_per_array == 4


@pytest.mark.parametrize("kwargs", [
    dict(activation_bits=1), dict(weight_bits=33), dict(activation_bits=True),
    dict(input_slice=(2, 6)), dict(input_slice=(1, 6)), dict(weight_slice=(1, 1, 1)),
    dict(input_slice=(1, 0, 7)), dict(adc_bits=0), dict(adc_bits=(6, 6)), dict(adc_bits=17),
    dict(array_size=(64, 62)), dict(array_size=(64,)), dict(rows_per_read=65),
    dict(seed=-1), dict(seed=2**32), dict(high_conductance=1e-7, low_conductance=1e-5),
    dict(read_voltage=0.0), dict(weight_quant_gran=(20, 1)), dict(input_quant_gran=(1, 40)),
    dict(bw_e=1), dict(bw_e=4, weight_signed=False), dict(weight_signed=1),
    dict(low_conductance=float("nan")), dict(high_conductance=1e39),
    dict(activation_bits=32, weight_bits=32, adc_bits=16),
])
def test_invalid_configs_raise(kwargs):
    with pytest.raises((ValueError, TypeError)):
        Config(**kwargs)


def test_read_alignment_rules():
    Config(array_size=(64, 64), rows_per_read=16, weight_quant_gran=(32, 1))
    Config(array_size=(64, 64), rows_per_read=16, input_quant_gran=(1, 128))
    with pytest.raises(ValueError):
        Config(array_size=(64, 64), rows_per_read=24, weight_quant_gran=(48, 1))


def test_nonidealities_validation():
    Nonidealities(stuck_at_low=0.5, stuck_at_high=0.5)
    for kwargs in (dict(write_variation=-1), dict(read_mode="bogus"),
                   dict(stuck_at_low=0.7, stuck_at_high=0.4), dict(drift_reference_time=0),
                   dict(read_variation=float("inf")), dict(write_variation=True)):
        with pytest.raises(ValueError):
            Nonidealities(**kwargs)


def test_config_hashable_and_frozen():
    a, b = Config(**BASELINE), Config(**BASELINE)
    assert a == b and hash(a) == hash(b)
    with pytest.raises(Exception):
        a.seed = 1


def test_int64_bound_matches_formula():
    for bits, adc in itertools.product((8, 16, 32), (6, 16)):
        kwargs = dict(activation_bits=bits, weight_bits=bits, adc_bits=adc)
        layout_a = oracle._layout(None, bits)
        maxima = [(1 << adc) - 1] * bits
        bound = sum(abs(f) for _, _, f in layout_a) * sum(abs(f) * m for (_, _, f), m in
                                                           zip(layout_a, maxima))
        if bound > 2**63 - 1:
            with pytest.raises(ValueError):
                Config(**kwargs)
        else:
            assert Config(**kwargs).reconstruction_bound == bound
