"""Benchmark: Simulator.mm at M=N=K=4096, INT8 (1,1,2,2,2) slices, on one MI355X.

Workload: A, B = randn(4096, 4096) (seed 135), array
128x128, rows_per_read 32, groups (32,1)/(1,32), adc_bits (6,7,7,8,8).  A step
is one full ``Simulator.mm(A, B)`` on resident HBM inputs with ideal devices:
input quantization, RHS re-programming (as the reference does every call),
the fused MFMA read and the finiteness checks.  The noisy variant (write 0.02,
shared read 0.01, S-curve ADC alpha 0.1) is timed alongside.

Prints one JSON line.  ``value`` is effective GMAC/s (N*K*O per second);
``slice_mac_per_s`` counts the 25 slice pairs; ``roofline`` prices the fused
kernel's slice-MACs (2 ops each) against the dense int8 MFMA peak, with the
kernel duration measured by HIP events on its launch stream.
"""

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

SIZE = 4096
BASE = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
            weight_slice=(1, 1, 2, 2, 2), array_size=(128, 128), rows_per_read=32,
            weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=(6, 7, 7, 8, 8))
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, tera-ops/s
HBM_PEAK_GBS = 8000.0

# HBM bytes per launch of the read kernel on this workload, from two rocprofv3
# --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch) scaled by what the
# same counters read for a 256 MiB device copy (FETCH x1.99974, WRITE x1.0):
# 225.1 MiB read + 64.0 MiB written.  Summary and commands:
# profiles/k_ideal_config2_pmc.md.  Only valid for the kernel sources it was
# measured on (hash prefix below); otherwise the bench reports null.
MEASURED_TRAFFIC = dict(kernels="ce3a6329d20ce4c8", bytes=303186787)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def time_steps(fn, steps, warmup):
    import torch

    from memfast_amd import hip

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    hip.collect_kernel_times()
    hip.profile_kernels(True)
    start = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    hip.profile_kernels(False)
    launches, total_ms = hip.collect_kernel_times()
    return elapsed / steps * 1e3, total_ms / max(1, launches)


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--noisy-steps", type=int, default=2)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                        help="first run one device-to-device copy of MIB MiB (a known-size "
                             "kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the sliced matmul path is built and measured on a "
              "single MI355X (column-tile sharding across GPUs is described in DESIGN.md but "
              "not run); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import memfast_amd as memfast
    from memfast_amd import hip

    device = torch.device("cuda", 0)
    torch.manual_seed(135)
    a_cpu = torch.randn(SIZE, SIZE)
    b_cpu = torch.randn(SIZE, SIZE)
    a = a_cpu.to(device)
    b = b_cpu.to(device)
    if args.copy_calibration > 0:
        source = torch.ones(args.copy_calibration << 20, dtype=torch.uint8, device=device)
        torch.empty_like(source).copy_(source)
        torch.cuda.synchronize()
        del source
    ideal_cfg = memfast.Config(**BASE, nonidealities=memfast.Nonidealities(write_variation=0.0))
    sim = memfast.Simulator(ideal_cfg, device=device)
    ms_step, kernel_ms = time_steps(lambda: sim.mm(a, b), args.steps, args.warmup)

    macs = SIZE**3
    pairs = len(ideal_cfg.input_layout) * len(ideal_cfg.weight_layout)
    slice_macs = macs * pairs
    value = macs / (ms_step * 1e-3) / 1e9
    achieved = 2 * slice_macs / (kernel_ms * 1e-3) / 1e12

    noisy = None
    if args.noisy_steps > 0:
        noisy_cfg = memfast.Config(**BASE, nonidealities=memfast.Nonidealities(
            write_variation=0.02, read_variation=0.01, adc_nonlinearity=0.1))
        noisy_sim = memfast.Simulator(noisy_cfg, device=device)
        noisy_ms, noisy_kernel_ms = time_steps(lambda: noisy_sim.mm(a, b), args.noisy_steps, 1)
        noisy = dict(ms_per_step=round(noisy_ms, 3), kernel_ms=round(noisy_kernel_ms, 3),
                     value=round(macs / (noisy_ms * 1e-3) / 1e9, 3), unit="GMAC/s",
                     config="write_variation=0.02, read_variation=0.01 shared, "
                            "adc_nonlinearity=0.1")

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        threads = os.cpu_count()
        torch.set_num_threads(threads)
        rows, cols = 1024, 256
        start = time.perf_counter()
        oracle.mm(a_cpu[:rows], b_cpu[:, :cols], ideal_cfg)
        seconds = time.perf_counter() - start
        cpu = dict(
            value=rows * cols * SIZE / seconds / 1e9,
            unit="GMAC/s",
            cores=torch.get_num_threads(),
            kind="port",
            sample=(f"oracle.mm(A[:{rows}], B[:, :{cols}]) at K={SIZE} (one two-tile chunk of "
                    f"a quarter of the rows), ideal devices, {seconds:.2f} s on "
                    f"{threads} threads of {cpu_model()}"),
        )

    kernels = hip.native_source_hash()[:16]
    traffic = MEASURED_TRAFFIC["bytes"] if MEASURED_TRAFFIC["kernels"] == kernels else None
    line = dict(
        metric="effective GMAC/s, Simulator.mm 4096^3 INT8 (1,1,2,2,2)",
        value=round(value, 3),
        unit="GMAC/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        ms_per_step=round(ms_step, 4),
        higher_is_better=True,
        scaling="weak",
        vs_baseline=None,
        dtype="int8",
        data="synthetic",
        config=dict(
            workload="Simulator.mm A[4096,4096] @ B[4096,4096], ideal devices, BASELINE config 2",
            M=SIZE, K=SIZE, O=SIZE, array_size=[128, 128], rows_per_read=32,
            slices="(1,1,2,2,2)x(1,1,2,2,2)", adc_bits=[6, 7, 7, 8, 8], kernel="ideal MFMA",
        ),
        slice_mac_per_s=slice_macs / (ms_step * 1e-3),
        kernel_ms=round(kernel_ms, 4),
        roofline=dict(bound="mfma", achieved=round(achieved, 2), peak=INT8_PEAK_TOPS,
                      unit="TFLOP/s", frac=round(achieved / INT8_PEAK_TOPS, 4), traffic=traffic,
                      note="int8 tera-ops (2 per slice-MAC, 25 pairs) / read-kernel time "
                           "(HIP events on its stream); traffic = HBM bytes per launch"),
        noisy=noisy,
        cpu_baseline=cpu,
        kernels=kernels,
    )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
