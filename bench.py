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
FP16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, TFLOP/s (the noisy read's precision)
HBM_PEAK_GBS = 8000.0

# HBM bytes per launch of the read kernels on this workload (ideal: k_ideal; noisy:
# k_noisy), from two rocprofv3 --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB per
# dispatch) scaled by what the same counters read for a 256 MiB device copy in the same
# runs.  Summaries and commands: profiles/k_ideal_config2_pmc.md and
# profiles/k_noisy_config2_noisy_pmc.md.  Only valid for the kernel sources they were
# measured on (hash prefix below); otherwise the bench reports null.
MEASURED_TRAFFIC = dict(kernels="189a79d1c78a7483", ideal=298991309, noisy=2054246156)


def measured_traffic(leg):
    """HBM bytes per launch of the leg's read kernel, if measured on these kernel sources."""
    from memfast_amd import hip

    if MEASURED_TRAFFIC["kernels"] != hip.native_source_hash()[:16]:
        return None
    return MEASURED_TRAFFIC[leg]


def progress(message):
    """One line per finished leg on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {message}", file=sys.stderr, flush=True)


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


def timed(fn, repeats=1):
    """Seconds per call of fn (after one untimed call), synchronized."""
    import torch

    fn()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(repeats):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - start) / repeats


def resnet18():
    """ResNet-18 (BasicBlock [2, 2, 2, 2], 1000 classes), Kaiming-normal conv init."""
    from torch import nn

    class Block(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
            self.bn1 = nn.BatchNorm2d(cout)
            self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
            self.bn2 = nn.BatchNorm2d(cout)
            self.down = None
            if stride != 1 or cin != cout:
                self.down = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False),
                                          nn.BatchNorm2d(cout))

        def forward(self, x):
            out = self.bn1(self.conv1(x)).relu()
            out = self.bn2(self.conv2(out))
            return (out + (x if self.down is None else self.down(x))).relu()

    layers = [nn.Conv2d(3, 64, 7, 2, 3, bias=False), nn.BatchNorm2d(64), nn.ReLU(),
              nn.MaxPool2d(3, 2, 1)]
    cin = 64
    for cout, stride in ((64, 1), (128, 2), (256, 2), (512, 2)):
        layers += [Block(cin, cout, stride), Block(cout, cout, 1)]
        cin = cout
    layers += [nn.AdaptiveAvgPool2d(1), nn.Flatten(), nn.Linear(512, 1000)]
    model = nn.Sequential(*layers)
    for module in model.modules():
        if isinstance(module, nn.Conv2d):
            nn.init.kaiming_normal_(module.weight, mode="fan_out", nonlinearity="relu")
    return model.eval()


def secondary(device, only=None):
    """The other BASELINE configurations, one timed run each (latency or throughput);
    ``only`` (a set of result names) restricts the run to those configurations."""
    def want(name):
        return only is None or name in only

    out = {}
    int8 = dict(activation_bits=8, weight_bits=8, input_slice=(1, 1, 2, 2, 2),
                weight_slice=(1, 1, 2, 2, 2))
    legs = [("config1_readme_mm", lambda: _config1(out, int8, device)),
            ("config3_gru", lambda: _config3(out, int8, device)),
            ("config4_resnet18", lambda: _config4(out, int8, device)),
            ("config5_llm_q_proj", lambda: _config5(out, device)),
            ("ideal_input_cases", lambda: _ideal_input_cases(out, device)),
            ("read_modes_general", lambda: _read_modes(out, device))]
    for name, run in legs:
        if want(name):
            run()
            progress(f"{name} done")
    return out


def _ideal_input_cases(out, device):
    """Config 2 (ideal) on inputs that defeat the ideal kernel's clamp-free proofs: ReLU-like
    A (every code nonnegative) and saturating +-1 operands (every code +-127, digits dense)."""
    import torch

    import memfast_amd as memfast

    cfg = memfast.Config(**BASE, nonidealities=memfast.Nonidealities(write_variation=0.0))
    gen = torch.Generator(device=device).manual_seed(137)
    cases = {
        "relu_a": (torch.randn(SIZE, SIZE, device=device, generator=gen).relu(),
                   torch.randn(SIZE, SIZE, device=device, generator=gen)),
        "saturating": (torch.randn(SIZE, SIZE, device=device, generator=gen).sign(),
                       torch.randn(SIZE, SIZE, device=device, generator=gen).sign()),
    }
    pairs = len(cfg.input_layout) * len(cfg.weight_layout)
    for name, (a, b) in cases.items():
        sim = memfast.Simulator(cfg, device=device)
        ms, kernel_ms = time_steps(lambda: sim.mm(a, b), 5, 1)
        tops = 2 * SIZE**3 * pairs / (kernel_ms * 1e-3) / 1e12
        out[f"ideal_{name}"] = dict(ms_per_step=round(ms, 3), kernel_ms=round(kernel_ms, 3),
                                    gmac_per_s=round(SIZE**3 / (ms * 1e-3) / 1e9, 1),
                                    frac=round(tops / INT8_PEAK_TOPS, 4))


def _read_modes(out, device):
    """Config 2's array shape at 4096^3 with the other noise forms, all on the noisy MFMA
    read: per-slice-pair read noise (a plane of terms per input slice), output-mode read
    noise (mean and variance sums, a normal per conversion), voltage noise (real input
    operands) and output-mode read noise with voltage noise (real operands and their
    squares); then config 5's wide slicing, and FP64 currents."""
    import torch

    import memfast_amd as memfast
    from memfast_amd import hip

    torch.manual_seed(135)
    a = torch.randn(SIZE, SIZE, device=device)
    b = torch.randn(SIZE, SIZE, device=device)
    modes = {
        "slice_pair": dict(write_variation=0.02, read_variation=0.01, read_mode="slice_pair"),
        "output": dict(write_variation=0.02, read_variation=0.01, read_mode="output"),
        "voltage": dict(write_variation=0.02, voltage_variation=0.01),
        "output_voltage": dict(write_variation=0.02, read_variation=0.01, read_mode="output",
                               voltage_variation=0.01),
    }
    for name, effects in modes.items():
        cfg = memfast.Config(**BASE, nonidealities=memfast.Nonidealities(**effects))
        kernel = hip.mm_kernel(cfg, SIZE, SIZE // 128, SIZE // 128)
        sim = memfast.Simulator(cfg, device=device)
        steps = 5 if kernel else 1
        ms, kernel_ms = time_steps(lambda: sim.mm(a, b), steps, 1)
        out[f"read_mode_{name}"] = dict(ms_per_step=round(ms, 2), kernel_ms=round(kernel_ms, 2),
                                        gmac_per_s=round(SIZE**3 / (ms * 1e-3) / 1e9, 1),
                                        kernel={0: "general FP32", 2: "noisy MFMA"}[kernel])
    # Wide codes (config 5's slicing: BFP16 x INT4, nine input and three weight slices,
    # 64x64 arrays) at the same size, on the wide MFMA read: shared read noise, voltage
    # variation (real input operands) and slice_pair read noise (a plane of terms per
    # input slice, read from global memory).
    wide = dict(activation_bits=16, weight_bits=4, input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2),
                weight_slice=(1, 1, 2), bw_e=8, adc_bits=(6, 6, 7))
    shared = dict(read_variation=0.01, drift_coefficient=0.05, drift_time=100.0)
    wide_modes = {
        "wide_shared": shared,
        "wide_voltage": shared | dict(voltage_variation=0.01),
        "wide_slice_pair": shared | dict(read_mode="slice_pair"),
    }
    for name, effects in wide_modes.items():
        cfg = memfast.Config(**wide, nonidealities=memfast.Nonidealities(**effects))
        kernel = hip.mm_kernel(cfg, SIZE, SIZE // 64, SIZE // 64)
        assert kernel == 3, (name, kernel)
        sim = memfast.Simulator(cfg, device=device)
        ms, kernel_ms = time_steps(lambda: sim.mm(a, b), 3, 1)
        out[f"read_mode_{name}"] = dict(ms_per_step=round(ms, 2), kernel_ms=round(kernel_ms, 2),
                                        gmac_per_s=round(SIZE**3 / (ms * 1e-3) / 1e9, 1),
                                        kernel="wide MFMA")
    # FP64 currents (precise_currents: high - low = 5e-5 of high) at config 2's slicing and
    # size, on the FP64 MFMA read, with write and shared read noise.
    cfg = memfast.Config(**BASE, high_conductance=1e-5, low_conductance=9.9995e-6,
                         nonidealities=memfast.Nonidealities(write_variation=2e-6,
                                                             read_variation=1e-6))
    assert cfg.precise_currents and hip.mm_kernel(cfg, SIZE, SIZE // 128, SIZE // 128) == 0
    sim = memfast.Simulator(cfg, device=device)
    ms, kernel_ms = time_steps(lambda: sim.mm(a, b), 3, 1)
    out["read_mode_precise"] = dict(ms_per_step=round(ms, 2), kernel_ms=round(kernel_ms, 2),
                                    gmac_per_s=round(SIZE**3 / (ms * 1e-3) / 1e9, 1),
                                    kernel="FP64 MFMA")


def _config1(out, int8, device):
    import torch

    import memfast_amd as memfast

    # Config 1: README first simulation (4x128 @ 128x32, write variation).
    cfg = memfast.Config(**int8, array_size=(128, 128), rows_per_read=32,
                         weight_quant_gran=(32, 1), input_quant_gran=(1, 32), adc_bits=7,
                         nonidealities=memfast.Nonidealities(write_variation=0.02))
    torch.manual_seed(135)
    a, b = torch.randn(4, 128, device=device), torch.randn(128, 32, device=device)
    sim = memfast.Simulator(cfg, device=device)
    seconds = timed(lambda: sim.mm(a, b), 50)
    out["config1_readme_mm"] = dict(us_per_call=round(seconds * 1e6, 1), macs=4 * 128 * 32)


def _config3(out, int8, device):
    import torch
    from torch import nn

    import memfast_amd as memfast

    # Config 3: converted 1-layer GRU (40 -> 512), batch 32, 200 steps.
    cfg = memfast.Config(**int8, array_size=(128, 128), rows_per_read=32, adc_bits=7,
                         nonidealities=memfast.Nonidealities(write_variation=0.02))
    torch.manual_seed(135)
    gru = nn.GRU(40, 512, 1).to(device)
    analog = memfast.convert_model(gru, memfast.Simulator(cfg, device=device))
    x = torch.randn(200, 32, 40, device=device)
    seconds = timed(lambda: analog(x))
    macs = 200 * 32 * (40 + 512) * 3 * 512
    out["config3_gru"] = dict(ms_per_sequence=round(seconds * 1e3, 2),
                              us_per_step=round(seconds / 200 * 1e6, 1),
                              gmac_per_s=round(macs / seconds / 1e9, 2))


def _config4(out, int8, device):
    import torch
    from torch import nn

    import memfast_amd as memfast

    # Config 4: ResNet-18, batch 64 at 224^2, every Conv2d/Linear converted, fixed input
    # scales from a 4-batch synthetic calibration, write variation + 0.1% stuck-at faults.
    cfg = memfast.Config(**int8, array_size=(256, 256), rows_per_read=64,
                         weight_quant_gran=(None, 1), adc_bits=8,
                         nonidealities=memfast.Nonidealities(write_variation=0.02,
                                                             stuck_at_low=0.0005,
                                                             stuck_at_high=0.0005))
    torch.manual_seed(135)
    model = resnet18().to(device)
    maxima = {}
    hooks = [module.register_forward_pre_hook(
        lambda module, inputs, name=name: maxima.__setitem__(
            name, max(maxima.get(name, 0.0), float(inputs[0].detach().abs().amax()))))
        for name, module in model.named_modules() if isinstance(module, (nn.Conv2d, nn.Linear))]
    with torch.no_grad():
        for _ in range(4):
            model(torch.randn(16, 3, 224, 224, device=device))
    for hook in hooks:
        hook.remove()
    analog = memfast.convert_model(model, memfast.Simulator(cfg, device=device))
    upper = (1 << (cfg.activation_bits - 1)) - 1
    for name, module in analog.named_modules():
        if name in maxima:
            scale = max(maxima[name] if maxima[name] > 0 else 1.0, 1.1754943508222875e-38) / upper
            matrices = module.matrices if hasattr(module, "matrices") else [module]
            for matrix in matrices:
                matrix.set_input_scale(scale)
    images = torch.randn(64, 3, 224, 224, device=device)
    with torch.no_grad():
        seconds = timed(lambda: analog(images))
    out["config4_resnet18"] = dict(ms_per_batch=round(seconds * 1e3, 1), batch=64,
                                   images_per_s=round(64 / seconds, 1),
                                   gmac_per_s=round(116.0e9 / seconds / 1e9, 1))


def _config5(out, device):
    import torch

    import memfast_amd as memfast

    # Config 5 (sample): one q_proj 4096x4096 on 2048 tokens, BFP bw_e=8 16-bit inputs
    # (1,1,2,2,2,2,2,2,2) x INT4 weights (1,1,2), drift + read noise; default schedule.
    cfg = memfast.Config(activation_bits=16, weight_bits=4,
                         input_slice=(1, 1, 2, 2, 2, 2, 2, 2, 2), weight_slice=(1, 1, 2),
                         bw_e=8, adc_bits=(6, 6, 7),
                         nonidealities=memfast.Nonidealities(read_variation=0.01,
                                                             drift_coefficient=0.05,
                                                             drift_time=100.0))
    torch.manual_seed(135)
    tokens = torch.randn(2048, 4096, device=device)
    tokens[:, torch.randperm(4096, device=device)[:41]] *= 20   # 1% outlier channels
    weight = torch.randn(4096, 4096, device=device) * 0.02
    sim = memfast.Simulator(cfg, device=device)
    seconds = timed(lambda: sim.mm(tokens, weight), 3)
    out["config5_llm_q_proj"] = dict(ms_per_call=round(seconds * 1e3, 1), tokens=2048,
                                     gmac_per_s=round(2048 * 4096 * 4096 / seconds / 1e9, 2))
    # BASELINE config 5 names tuned mode: the first call searches the wide read's LDS tiers
    # (bit-exact against the default schedule) and caches the winner; later calls reuse it.
    import tempfile

    with tempfile.TemporaryDirectory() as cache:
        tuned = memfast.Simulator(cfg, device=device, mode="tuned", cache_dir=cache)
        start = time.perf_counter()
        tuned.mm(tokens, weight)
        torch.cuda.synchronize()
        search = time.perf_counter() - start
        tuned_seconds = timed(lambda: tuned.mm(tokens, weight), 3)
        record = tuned.report()["selections"][0]
    out["config5_llm_q_proj"].update(
        tuned_ms_per_call=round(tuned_seconds * 1e3, 2), tuning_seconds=round(search, 3),
        tuned_selected=dict(tier=record["selected"]["tier"], kernel=record["kernel"]),
        tuned_candidates={str(c["schedule"]["tier"]): round(c["seconds"] * 1e3, 3)
                          for c in record["candidates"] if c["status"] == "accepted"})


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--noisy-steps", type=int, default=2)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-secondary", action="store_true",
                        help="skip the timing of BASELINE configurations 1, 3, 4 and 5")
    parser.add_argument("--secondary-only", default=None, metavar="NAMES",
                        help="time only these secondary configurations (comma-separated result "
                             "names, e.g. config4_resnet18) and print them; for profiling")
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
    if args.copy_calibration > 0:
        source = torch.ones(args.copy_calibration << 20, dtype=torch.uint8, device=device)
        torch.empty_like(source).copy_(source)
        torch.cuda.synchronize()
        del source
    if args.secondary_only:
        names = set(args.secondary_only.split(","))
        print(json.dumps(dict(secondary=secondary(device, only=names))), flush=True)
        return
    torch.manual_seed(135)
    a_cpu = torch.randn(SIZE, SIZE)
    b_cpu = torch.randn(SIZE, SIZE)
    a = a_cpu.to(device)
    b = b_cpu.to(device)
    ideal_cfg = memfast.Config(**BASE, nonidealities=memfast.Nonidealities(write_variation=0.0))
    sim = memfast.Simulator(ideal_cfg, device=device)
    ms_step, kernel_ms = time_steps(lambda: sim.mm(a, b), args.steps, args.warmup)
    progress(f"ideal leg: {ms_step:.3f} ms per step")

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
        progress(f"noisy leg: {noisy_ms:.3f} ms per step")
        noisy_achieved = 2 * slice_macs / (noisy_kernel_ms * 1e-3) / 1e12
        noisy = dict(
            ms_per_step=round(noisy_ms, 3), kernel_ms=round(noisy_kernel_ms, 3),
            value=round(macs / (noisy_ms * 1e-3) / 1e9, 3), unit="GMAC/s",
            config="write_variation=0.02, read_variation=0.01 shared, adc_nonlinearity=0.1",
            roofline=dict(bound="mfma", achieved=round(noisy_achieved, 2), peak=FP16_PEAK_TFLOPS,
                          unit="TFLOP/s", frac=round(noisy_achieved / FP16_PEAK_TFLOPS, 4),
                          traffic=measured_traffic("noisy"),
                          note="2 flops per slice-MAC (25 pairs) / k_noisy time (HIP events "
                               "on its stream, the conductance split excluded); the hardware "
                               "issues two fp16 MFMAs (hi and lo conductance terms) per "
                               "slice-MAC, twice this count"),
        )

    others = None if args.no_secondary else secondary(device)

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle

        threads = os.cpu_count()
        torch.set_num_threads(threads)
        rows, cols = 4096, 256   # about 10 s on 16 threads
        start = time.perf_counter()
        oracle.mm(a_cpu[:rows], b_cpu[:, :cols], ideal_cfg)
        seconds = time.perf_counter() - start
        progress(f"cpu baseline: {seconds:.1f} s")
        cpu = dict(
            value=rows * cols * SIZE / seconds / 1e9,
            unit="GMAC/s",
            cores=torch.get_num_threads(),
            kind="port",
            sample=(f"oracle.mm(A[:{rows}], B[:, :{cols}]) at K={SIZE} (one two-tile chunk of "
                    f"every row), ideal devices, {seconds:.2f} s on "
                    f"{threads} threads of {cpu_model()}"),
        )

    kernels = hip.native_source_hash()[:16]
    traffic = measured_traffic("ideal")
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
        secondary=others,
        kernels=kernels,
    )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
