"""Write golden vectors from the reference's own CPU path (run in the build container only).

Imports HUST-ISMD-Odyssey/MemFast 0.3.0 from /root/reference (pure Python +
torch CPU) to record input/output vectors for the parts of the oracle that no
closed form, checkpoint fixture or brute force pins:
  * the counter-based RNG (memfast/random.py:8-33): uniform / normal samples
    for hand-picked addresses (including >= 2^32), seeds and streams, and
    event seeds;
  * noisy array reads: restored conductances, slice totals and full
    Simulator.mm outputs on CPU for small shapes under every device effect.
The reference never travels: only the vectors in reference_vectors.npz are
committed.  Run: python tests/golden/make_reference_vectors.py
"""

import json
import sys
from pathlib import Path

import numpy as np
import torch

REFERENCE = Path("/root/reference")
OUT = Path(__file__).with_name("reference_vectors.npz")


def cases():
    """(name, Config kwargs, Nonidealities kwargs, N, K, O) for the noisy sweep."""
    base = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                weight_quant_gran=(16, 1), input_quant_gran=(1, 16), adc_bits=(6, 7, 7, 8, 8))
    return [
        ("ideal", base, dict(write_variation=0.0), 5, 70, 40),
        ("write", base, dict(write_variation=0.02), 5, 70, 40),
        ("shared", base, dict(write_variation=0.02, read_variation=0.01,
                              adc_nonlinearity=0.1), 5, 70, 40),
        ("slice_pair", base, dict(write_variation=0.02, read_variation=0.02,
                                  read_mode="slice_pair"), 4, 64, 33),
        ("output", base, dict(write_variation=0.02, read_variation=0.02, read_mode="output"),
         4, 64, 33),
        ("voltage", base, dict(write_variation=0.0, voltage_variation=0.05), 4, 64, 33),
        ("saf_drift", base, dict(write_variation=0.02, stuck_at_low=0.05, stuck_at_high=0.03,
                                 drift_coefficient=0.05, drift_time=100.0), 4, 64, 33),
        ("binary_int4", dict(activation_bits=8, weight_bits=4, array_size=(64, 64),
                             adc_bits=6), dict(write_variation=0.02), 3, 150, 20),
        # Wide configurations (FP64 scales and restore, 64-bit codes, BFP).
        ("bfp16_int4", dict(activation_bits=16, weight_bits=4,
                            input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2), weight_slice=(1, 1, 2),
                            bw_e=8, array_size=(64, 64), adc_bits=(6, 6, 7)),
         dict(write_variation=0.02, read_variation=0.01, drift_coefficient=0.05,
              drift_time=100.0), 3, 150, 20),
        ("int12_ideal", dict(activation_bits=12, weight_bits=10, array_size=(32, 16),
                             rows_per_read=16, adc_bits=8), dict(write_variation=0.0), 3, 70, 24),
        ("bfp8_binary", dict(activation_bits=8, weight_bits=8, bw_e=4, array_size=(32, 16),
                             rows_per_read=16, adc_bits=6),
         dict(write_variation=0.02, adc_nonlinearity=0.05), 4, 64, 33),
        # FP64 currents (memfast/config.py:215-224, `precise_currents`): a 9-bit input
        # slice (mask 511 > 255, wide codes) ...
        ("precise_slice9_ideal", PRECISE_SLICE9, dict(write_variation=0.0), 3, 70, 24),
        ("precise_slice9", PRECISE_SLICE9,
         dict(write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1), 3, 70, 24),
        # ... and narrow INT8 codes with high - low < 1e-4 * high, where FP32 conductance
        # differences lose the count; the noise is scaled to a few percent of high - low.
        ("precise_close_ideal", PRECISE_CLOSE, dict(write_variation=0.0), 4, 64, 33),
        ("precise_close", PRECISE_CLOSE,
         dict(write_variation=2e-6, read_variation=1e-6, adc_nonlinearity=0.1), 4, 64, 33),
    ]


PRECISE_SLICE9 = dict(activation_bits=12, weight_bits=8, input_slice=(1, 2, 9),
                      weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                      adc_bits=8)
PRECISE_CLOSE = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                     weight_slice=(1, 1, 2, 2, 2), array_size=(32, 16), rows_per_read=16,
                     weight_quant_gran=(16, 1), input_quant_gran=(1, 16), adc_bits=(6, 7, 7, 8, 8),
                     high_conductance=1e-5, low_conductance=0.99995e-5)


def bfp_edge_values():
    """FP64 rows whose 4-wide group maxima sit at, just below and just above powers of two."""
    rows = []
    for k in (-30, -2, -1, 0, 1, 3, 7, 20, 100):
        top = 2.0 ** k
        for peak in (top * (1 - 2.0**-53), top, top * (1 + 2.0**-52), top * 1.5,
                     top * (1 - 2.0**-40)):
            rows.append([peak, -peak / 3, peak / 7, 0.0])
    return torch.tensor(rows, dtype=torch.float64).reshape(-1, 4)


def main():
    sys.path.insert(0, str(REFERENCE))
    import memfast
    from memfast import Config, Nonidealities, Simulator, reference
    from memfast import random as mrandom
    from memfast.quantization import input_tiles

    torch.manual_seed(135)
    vectors = {}
    # RNG ---------------------------------------------------------------
    addresses = torch.tensor(
        [0, 1, 2, 3, 12345, 2**31 - 1, 2**31, 2**32 - 1, 2**32, 2**32 + 7, 3 * 2**32 + 11,
         2**40 + 5, 2**47 - 3, 2**52 + 99, 2**62 + 12345, 2**63 - 1],
        dtype=torch.int64,
    )
    addresses = torch.cat([addresses, torch.randint(0, 2**62, (48,), dtype=torch.int64)])
    seeds = [0, 135, 4017293833, 2**32 - 1, 0x1234567890ABCDEF & (2**63 - 1), 2**63 - 5]
    streams = [10, 20, 30, 40, 60]
    vectors["rng_address"] = addresses.numpy()
    vectors["rng_seeds"] = np.array(seeds, dtype=np.uint64)
    vectors["rng_streams"] = np.array(streams, dtype=np.int64)
    uni = np.zeros((len(seeds), len(streams), len(addresses)), np.float32)
    nor = np.zeros_like(uni)
    for si, seed in enumerate(seeds):
        for ti, stream in enumerate(streams):
            uni[si, ti] = mrandom.uniform(addresses, seed, stream).numpy()
            nor[si, ti] = mrandom.normal(addresses, seed, stream).numpy()
    vectors["rng_uniform"] = uni
    vectors["rng_normal"] = nor
    events = [0, 1, 2, 7, 2**31, 2**32 - 1, 2**32, 2**32 + 3, 2**40 + 17, 2**63 - 1]
    pairs = [(s, e) for s in (135, 4017293833, 2**32 - 1) for e in events]
    vectors["event_pairs"] = np.array(pairs, dtype=np.uint64)
    vectors["event_seeds"] = np.array([mrandom.event_seed(s, e) for s, e in pairs], dtype=np.uint64)
    vectors["mix_in"] = np.array([0, 1, 2, 0xDEADBEEF, 2**32 - 1, 123456789], dtype=np.uint64)
    vectors["mix_out"] = np.array(
        [int(mrandom.mix(torch.tensor(int(v)))) for v in vectors["mix_in"]], dtype=np.uint64
    )
    # Array reads ---------------------------------------------------------
    names = []
    for name, cfg_kwargs, ni_kwargs, n, k, o in cases():
        config = Config(**cfg_kwargs, nonidealities=Nonidealities(**ni_kwargs))
        a = torch.randn(n, k)
        b = torch.randn(k, o)
        sim = Simulator(config, device="cpu")
        out0 = sim.mm(a, b)          # matrix.0, event 0
        out1 = sim.mm(a, b)          # same program, event 1
        matrix = sim._matrix_for(b)
        q, xscale = input_tiles(a, config)
        raw, _, _ = reference.restored(matrix.packed, config, matrix.seed, 0, 0, matrix.p)
        totals = reference.partial(q, matrix.packed, config, None, matrix.seed, 0, 0, matrix.p)
        prefix = f"case_{name}_"
        vectors[prefix + "config"] = np.array(json.dumps(dict(config=cfg_kwargs,
                                                              nonidealities=ni_kwargs)))
        vectors[prefix + "a"] = a.numpy()
        vectors[prefix + "b"] = b.numpy()
        vectors[prefix + "out0"] = out0.numpy()
        vectors[prefix + "out1"] = out1.numpy()
        vectors[prefix + "packed"] = matrix.packed.numpy()
        vectors[prefix + "wscale"] = matrix.weight_scale.numpy()
        vectors[prefix + "q"] = q.numpy()
        vectors[prefix + "xscale"] = xscale.numpy()
        vectors[prefix + "restored"] = raw.numpy()
        vectors[prefix + "totals"] = totals.numpy()
        vectors[prefix + "seed"] = np.array(matrix.seed, dtype=np.uint64)
        names.append(name)
    vectors["case_names"] = np.array(names)
    # BFP exponents floor(log2(max)) at power-of-two edges (quantization.py:35-40).
    from memfast.quantization import grouped_quantize

    edges = bfp_edge_values()
    vectors["bfp_edges_in"] = edges.numpy()
    for bits, bw_e in ((16, 8), (12, 5), (8, 11)):
        code, scale = grouped_quantize(edges, bits, (1, 4), bw_e)
        vectors[f"bfp_edges_code_{bits}_{bw_e}"] = code.numpy()
        vectors[f"bfp_edges_scale_{bits}_{bw_e}"] = scale.numpy()
    vectors["reference_version"] = np.array(memfast.__version__)
    np.savez_compressed(OUT, **vectors)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
