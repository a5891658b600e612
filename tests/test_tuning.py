"""Tuned-mode grid and schedule encoding (host-side; the kernel selection and workspace
queries of libmemfast_hip.so need no GPU)."""

import pytest

from memfast_amd import Config, Nonidealities, hip, tuning

INT8 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
            weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))
CONFIG5 = dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
               weight_slice=(1, 1, 2), bw_e=8, adc_bits=(6, 6, 7))


def test_grid_follows_the_selected_kernel():
    ideal = Config(**INT8, nonidealities=Nonidealities(write_variation=0.0))
    grid = tuning.schedule_grid(ideal, 4096, 32, arrays=32)
    assert [s["tile"] for s in grid] == ["64x64", "128x64"]
    rows64 = Config(**(INT8 | dict(rows_per_read=64, weight_quant_gran=(64, 1),
                                   input_quant_gran=(1, 64))),
                    nonidealities=Nonidealities(write_variation=0.0))
    assert [s["tile"] for s in tuning.schedule_grid(rows64, 4096, 32, arrays=32)] == ["64x64"]
    noisy = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02, read_variation=0.01))
    assert [s["split"] for s in tuning.schedule_grid(noisy, 64, 8, arrays=4)] == [0, 1, 2, 4, 8]
    assert [s["split"] for s in tuning.schedule_grid(noisy, 64, 8, arrays=1)] == [0, 1, 2, 4]
    wide = Config(**CONFIG5, nonidealities=Nonidealities(read_variation=0.01))
    assert [s["tier"] for s in tuning.schedule_grid(wide, 256, 4, arrays=8)] == [0, 1, 2, 3]
    slice_pair = Config(**INT8, nonidealities=Nonidealities(read_variation=0.01,
                                                             read_mode="slice_pair"))
    assert [s["split"] for s in tuning.schedule_grid(slice_pair, 64, 8, arrays=4)] == [
        0, 1, 2, 4, 8]
    # FP64 currents (high - low < 1e-4 high) run on the general kernel only.
    general = Config(**INT8, high_conductance=1e-5, low_conductance=0.99995e-5,
                     nonidealities=Nonidealities(write_variation=0.02))
    assert general.precise_currents and hip.mm_kernel(general, 64, 4, 8) == 0
    assert tuning.schedule_grid(general, 64, 8, arrays=4) == [tuning.default_schedule(general)]
    # Without the array count (the reference's signature) only the default is declared.
    assert tuning.schedule_grid(noisy, 64, 8) == [tuning.default_schedule(noisy)]
    for schedule in grid:
        assert {"arrays", "vectors", "columns", "workers"} <= set(schedule)


def test_schedule_variant_words():
    cfg = Config(**INT8)
    assert tuning.schedule_variant(tuning.default_schedule(cfg)) == tuning.DEFAULT_VARIANT == 2
    assert tuning.schedule_variant(dict(tile="128x64")) == 1
    assert tuning.schedule_variant(dict(split=4)) == 2 | 4 << 12
    assert tuning.schedule_variant(dict(tier=3)) == 2 | 3 << 16
    with pytest.raises(ValueError):
        hip.variant_word(split=16)
    with pytest.raises(ValueError):
        hip.variant_word(tier=4)


def test_workspace_need_prices_each_schedule():
    """A forced read split adds its integer totals (n * G * p * C * 4 bytes) to the noisy
    read's conductance terms; the ideal read needs only its digit masks; the general
    kernel with device noise needs the restored conductances."""
    noisy = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02))
    n, m, p = 256, 4, 8
    terms = tuning.workspace_need(noisy, n, m, p, dict(split=1))
    split = tuning.workspace_need(noisy, n, m, p, dict(split=2))
    assert split - terms == n * m * 4 * p * 128 * 4
    assert terms == (p * 128 // 64) * 2 * (5 * 32 * m * 128 * 2 * 2)
    ideal = Config(**INT8, nonidealities=Nonidealities(write_variation=0.0))
    assert tuning.workspace_need(ideal, n, m, p, {}) == (
        -(-(4 * 16 * 8) // 256) * 256 + -(-(32 * 16 * 8) // 256) * 256)
    # FP64 currents (general kernel): FP64 restored conductances.
    general = Config(**INT8, high_conductance=1e-5, low_conductance=0.99995e-5,
                     nonidealities=Nonidealities(write_variation=0.02))
    assert tuning.workspace_need(general, n, m, p, {}) == 8 * m * p * 5 * 128 * 128
    # Voltage variation adds the noisy read's input operands: hi and lo fp16 per input
    # slice, vector and physical row; with output-mode read noise also hi and lo of their
    # squares (and two planes of conductance terms).
    voltage = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02,
                                                          voltage_variation=0.01))
    assert tuning.workspace_need(voltage, n, m, p, dict(split=1)) == terms + 2 * 5 * n * m * 128 * 2
    output = Config(**INT8, nonidealities=Nonidealities(write_variation=0.02, read_variation=0.01,
                                                         read_mode="output",
                                                         voltage_variation=0.01))
    assert tuning.workspace_need(output, n, m, p, dict(split=1)) == 2 * terms + 4 * 5 * n * m * 128 * 2


def test_unknown_variant_bits_are_refused():
    import ctypes as ct

    cfg = Config(**INT8)
    size = ct.c_int64()
    rc = hip.library().mf_mm_workspace(ct.byref(hip.descriptor(cfg)), 64, 4, 8, 1 << 24,
                                       ct.byref(size))
    assert rc == hip.E_INVALID and b"variant" in hip.library().mf_last_error()
