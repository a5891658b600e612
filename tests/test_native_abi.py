"""The C-ABI library loads on any host and exports every symbol include/memfast_hip.h declares.

No compute call is made here (no GPU in the build container).
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from memfast_amd import hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "memfast_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(mf_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "mf_mm" in names and "mf_partial" in names and len(names) >= 14


def test_library_exports_every_declared_symbol():
    lib = hip.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(hip.LIBRARY)], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mf_\w+)", nm))
    assert set(declared_functions()) <= exported


def test_ctypes_signatures_cover_header():
    assert set(hip.SIGNATURES) == set(declared_functions())


def test_status_wait_reads_a_published_word():
    """mf_status_wait (host code only) returns the bits of a mailbox word that holds
    MF_STATUS_PUBLISHED and reports a word without it as unpublished after the timeout."""
    lib = hip.library()
    word = (ctypes.c_uint32 * 1)(0x80000000 | hip.STATUS_INPUT | hip.STATUS_RANGE)
    flags, published = ctypes.c_uint32(), ctypes.c_int32()
    assert lib.mf_status_wait(ctypes.addressof(word), 0, ctypes.byref(flags),
                              ctypes.byref(published)) == 0
    assert published.value == 1 and flags.value == hip.STATUS_INPUT | hip.STATUS_RANGE
    word[0] = hip.STATUS_WEIGHT   # bits without the published mark: not yet published
    assert lib.mf_status_wait(ctypes.addressof(word), 3000, ctypes.byref(flags),
                              ctypes.byref(published)) == 0
    assert published.value == 0 and flags.value == 0
    assert lib.mf_status_wait(None, 0, ctypes.byref(flags), ctypes.byref(published)) != 0


def test_abi_version_and_hash():
    lib = hip.library()
    assert lib.mf_abi_version() == hip.ABI_VERSION
    from memfast_amd.build_native import source_hash

    assert hip.native_source_hash() == source_hash(), "library is stale: rebuild it"


def test_struct_layout_matches_c(tmp_path):
    """Offsets of mf_config and mf_conv_geometry, sizes of mf_identity and mf_resources
    agree with gcc's."""
    fields = [name for name, _ in hip.MFConfig._fields_]
    geometry = [name for name, _ in hip.MFConvGeometry._fields_]
    probe = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(){"]
    lines += [f'printf("%zu\\n", offsetof(mf_config, {name}));' for name in fields]
    lines += [f'printf("%zu\\n", offsetof(mf_conv_geometry, {name}));' for name in geometry]
    lines += ['printf("%zu\\n%zu\\n%zu\\n%zu\\n", sizeof(mf_config), sizeof(mf_identity), '
              'sizeof(mf_resources), sizeof(mf_conv_geometry)); return 0;}']
    probe.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(probe)], check=True)
    values = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                             check=True).stdout.split()]
    offsets = [getattr(hip.MFConfig, name).offset for name in fields]
    offsets += [getattr(hip.MFConvGeometry, name).offset for name in geometry]
    assert values[:len(offsets)] == offsets
    assert values[len(offsets):] == [ctypes.sizeof(hip.MFConfig), ctypes.sizeof(hip.MFIdentity),
                                     ctypes.sizeof(hip.MFResources),
                                     ctypes.sizeof(hip.MFConvGeometry)]


def test_error_reporting_without_device():
    """Invalid descriptors are rejected on the host before any launch."""
    lib = hip.library()
    bad = hip.MFConfig()
    bad.abi_version = 999
    out = ctypes.c_int32()
    status = lib.mf_mm_kernel(ctypes.byref(bad), 1, 1, 1, 1, ctypes.byref(out))
    assert status == hip.E_INVALID
    assert b"ABI version" in lib.mf_last_error()
    with pytest.raises(ValueError):
        hip.check(status, "probe")


def test_descriptor_fp32_constants():
    import math
    import struct

    from memfast_amd import Config, Nonidealities

    cfg = Config(nonidealities=Nonidealities(read_variation=0.03, adc_nonlinearity=0.1))
    d = hip.descriptor(cfg)

    def f32(x):
        return struct.unpack("f", struct.pack("f", x))[0]

    assert d.f_span == f32(cfg.high_conductance - cfg.low_conductance)
    assert d.f_inv_unit == f32(1 / cfg.current_unit)
    assert d.f_two_pi == f32(2 * math.pi)
    assert d.f_out_mean == f32(math.expm1(0.5 * 0.03**2))
    assert list(d.adc_max)[:len(cfg.adc_maxima)] == list(cfg.adc_maxima)
    assert d.f_alpha_over_max[0] == f32(0.1 / cfg.adc_maxima[0])


def test_noisy_mfma_kernels_require_fp16_range():
    """The noisy MFMA reads hold k1*(g - L) in fp16; configurations whose sampled
    conductances could leave that range (huge noise, 8-bit weight slices with extreme
    variation) are routed to the general kernel by the host plan."""
    from memfast_amd import Config, Nonidealities
    base = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32)
    ok = Config(**base, nonidealities=Nonidealities(write_variation=0.02))
    assert hip.mm_kernel(ok, 64, 4, 4) == 2
    wild = Config(**base, nonidealities=Nonidealities(write_variation=3.0))
    assert hip.mm_kernel(wild, 64, 4, 4) == 0
    wide = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                  weight_slice=(1, 1, 2), bw_e=8, nonidealities=Nonidealities(read_variation=0.01))
    assert hip.mm_kernel(wide, 64, 4, 4) == 3
    wide_wild = Config(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                       weight_slice=(1, 1, 2), bw_e=8,
                       nonidealities=Nonidealities(read_variation=2.5))
    assert hip.mm_kernel(wide_wild, 64, 4, 4) == 0


def test_read_kernel_selection_by_noise_model():
    """Which read kernel each noise model takes (mf_mm_kernel, host only): the narrow noisy
    MFMA read covers voltage variation, slice_pair and output-mode read noise (also output
    mode with voltage variation); the wide MFMA read covers voltage variation and slice_pair
    read noise but not output-mode read noise (it models it not at all, so it must never
    reach it)."""
    from memfast_amd import Config, Nonidealities
    narrow = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                  weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32)
    wide = dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                weight_slice=(1, 1, 2), bw_e=8, array_size=(128, 128), rows_per_read=32)
    cases = [
        (narrow, dict(write_variation=0.02), 2),
        (narrow, dict(write_variation=0.02, voltage_variation=0.01), 2),
        (narrow, dict(read_variation=0.01, read_mode="slice_pair"), 2),
        (narrow, dict(read_variation=0.01, read_mode="output"), 2),
        (narrow, dict(read_variation=0.01, read_mode="output", voltage_variation=0.01), 2),
        (narrow, dict(read_variation=0.01, read_mode="slice_pair", voltage_variation=0.01), 2),
        (wide, dict(read_variation=0.01), 3),
        (wide, dict(write_variation=0.02, voltage_variation=0.01), 3),
        (wide, dict(read_variation=0.01, read_mode="slice_pair"), 3),
        (wide, dict(read_variation=0.01, read_mode="slice_pair", voltage_variation=0.01), 3),
        (wide, dict(read_variation=0.01, read_mode="output"), 0),
    ]
    for kwargs, effects, kernel in cases:
        cfg = Config(**kwargs, nonidealities=Nonidealities(**effects))
        assert hip.mm_kernel(cfg, 64, 4, 4) == kernel, (kwargs["activation_bits"], effects)
