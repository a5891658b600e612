"""ctypes binding of libmemfast_hip.so, the gfx950 accelerator backend.

Drop-in replacement of the reference's memfast/cuda.py (NVRTC + libcuda via
ctypes).  The Python-level names the simulator imports are kept:
``ResourceError`` (cuda.py:15-16), ``cache_root`` (:47-51), ``atomic_write``
(:54-64), ``program(...).resources(...)`` (:239-273, :313-319), ``partial``
(:322-373) and ``identity`` (:376-389).  Kernels are built ahead of time
(memfast_amd/build_native.py); physical constants travel in an ``mf_config``
descriptor instead of being compiled into the source.

There is no CPU fallback: every entry point raises when the library or a HIP
device is missing.
"""

import ctypes as ct
import math
import os
from functools import lru_cache
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "lib" / "libmemfast_hip.so"
MAX_SLICES = 32
ABI_VERSION = 9

OK, E_INVALID, E_UNSUPPORTED, E_RESOURCE, E_HIP = 0, 1, 2, 3, 4

READ_MODES = {"shared": 0, "slice_pair": 1, "output": 2}


class ResourceError(RuntimeError):
    """A launch exceeds a compiled kernel or device resource limit."""


class BackendError(RuntimeError):
    """The HIP backend is unavailable or a HIP runtime call failed."""


def cache_root():
    """Root of persistent caches: $MEMFAST_CACHE_DIR or $XDG_CACHE_HOME/memfast."""
    base = os.environ.get("MEMFAST_CACHE_DIR")
    if base:
        return Path(base).expanduser()
    return Path(os.environ.get("XDG_CACHE_HOME", Path.home() / ".cache")) / "memfast"


def atomic_write(path, content):
    """Write bytes through a temporary file in the same directory and rename."""
    import tempfile

    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.NamedTemporaryFile(dir=path.parent, delete=False) as stream:
        temporary = Path(stream.name)
        stream.write(content)
    try:
        os.replace(temporary, path)
    finally:
        temporary.unlink(missing_ok=True)


# ---------------------------------------------------------------------------
# C structures (include/memfast_hip.h)
# ---------------------------------------------------------------------------
class MFConfig(ct.Structure):
    _fields_ = [
        ("abi_version", ct.c_int32),
        ("rows", ct.c_int32), ("cols", ct.c_int32),
        ("read_rows", ct.c_int32), ("reads", ct.c_int32),
        ("activation_bits", ct.c_int32), ("weight_bits", ct.c_int32),
        ("weight_signed", ct.c_int32),
        ("n_in", ct.c_int32), ("n_w", ct.c_int32),
        ("in_shift", ct.c_int32 * MAX_SLICES), ("in_mask", ct.c_int32 * MAX_SLICES),
        ("in_factor", ct.c_int64 * MAX_SLICES),
        ("w_shift", ct.c_int32 * MAX_SLICES), ("w_mask", ct.c_int32 * MAX_SLICES),
        ("w_factor", ct.c_int64 * MAX_SLICES),
        ("adc_max", ct.c_int32 * MAX_SLICES),
        ("precise", ct.c_int32),
        ("read_mode", ct.c_int32),
        ("has_write", ct.c_int32), ("has_read", ct.c_int32), ("has_vnoise", ct.c_int32),
        ("has_nonlinear", ct.c_int32), ("has_saf", ct.c_int32), ("has_drift", ct.c_int32),
        ("f_high", ct.c_float), ("f_low", ct.c_float), ("f_voltage", ct.c_float),
        ("f_span", ct.c_float), ("f_inv_unit", ct.c_float),
        ("f_write", ct.c_float), ("f_read", ct.c_float), ("f_vnoise", ct.c_float),
        ("f_drift", ct.c_float),
        ("f_saf_low", ct.c_float), ("f_saf_band", ct.c_float),
        ("f_out_mean", ct.c_float), ("f_out_var", ct.c_float),
        ("f_two_pi", ct.c_float),
        ("f_alpha_over_max", ct.c_float * MAX_SLICES),
        ("d_high", ct.c_double), ("d_low", ct.c_double), ("d_voltage", ct.c_double),
        ("d_span", ct.c_double), ("d_inv_unit", ct.c_double), ("d_drift", ct.c_double),
        ("d_alpha_over_max", ct.c_double * MAX_SLICES),
        ("wide", ct.c_int32),
        ("bw_e", ct.c_int32),
    ]


class MFIdentity(ct.Structure):
    _fields_ = [
        ("arch", ct.c_char * 64),
        ("name", ct.c_char * 256),
        ("compute_units", ct.c_int32),
        ("driver_version", ct.c_int32),
        ("runtime_version", ct.c_int32),
        ("memory_bytes", ct.c_int64),
    ]


class MFResources(ct.Structure):
    _fields_ = [
        ("threads", ct.c_int32),
        ("shared_bytes", ct.c_int32),
        ("registers", ct.c_int32),
        ("local_bytes", ct.c_int32),
        ("max_blocks_per_cu", ct.c_int32),
    ]


class MFConvGeometry(ct.Structure):
    _fields_ = [(name, ct.c_int64) for name in (
        "n", "channels", "height", "width", "c0", "group_channels", "out_height", "out_width",
    )] + [(name, ct.c_int32) for name in ("kh", "kw", "sh", "sw", "ph", "pw", "dh", "dw")]


_P = ct.c_void_p
_I64 = ct.c_int64
_I32 = ct.c_int32
_CFG = ct.POINTER(MFConfig)

SIGNATURES = {
    "mf_abi_version": ([], _I32),
    "mf_last_error": ([], ct.c_char_p),
    "mf_source_hash": ([], ct.c_char_p),
    "mf_device_identity": ([ct.c_int, ct.POINTER(MFIdentity)], ct.c_int),
    "mf_input_tiles": ([_CFG, _P, _I64, _I64, _I64, _P, _P, _P, _P], ct.c_int),
    "mf_conv_input_tiles": ([_CFG, _P, ct.POINTER(MFConvGeometry), _P, _I64, _I64, _P, _P, _P,
                             _P, _P, _P], ct.c_int),
    "mf_quantize_inputs": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P],
                           ct.c_int),
    "mf_quantize_weights": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P,
                             _P], ct.c_int),
    "mf_transpose_packed": ([_CFG, _P, _I64, _I64, _P, _P], ct.c_int),
    "mf_restore": ([_CFG, _P, _I64, _I64, _I64, _I64, ct.c_uint32, ct.c_uint64, _P, _P],
                   ct.c_int),
    "mf_partial": ([_CFG, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, ct.c_uint32, ct.c_uint64,
                    _P, _P, _P], ct.c_int),
    "mf_mm": ([_CFG, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, ct.c_uint32,
               ct.c_uint64, _P, _I64, _P, _I64, _I32, _P, _P], ct.c_int),
    "mf_mm_from_float": ([_CFG, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P,
                          _P, _P, _P, _P, _P, _I64, _P, _I64, _I32, _P, _P, _P], ct.c_int),
    "mf_status_wait": ([_P, _I64, ct.POINTER(ct.c_uint32), ct.POINTER(_I32)], ct.c_int),
    "mf_status_publish": ([_P, _P, _P], ct.c_int),
    "mf_narrow_output": ([_P, _I64, _I64, _I64, _P, _P, _P], ct.c_int),
    "mf_mm_static": ([_CFG, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, ct.c_uint32,
                      ct.c_uint64, _P, _I64, _I32, _P, _P], ct.c_int),
    "mf_mm_totals": ([_CFG, _P, _I64, _I64, _P, _I64, _P, ct.c_uint32, ct.c_uint64, _P, _P, _I64,
                      _P], ct.c_int),
    "mf_bias_add": ([_P, _I64, _I64, _I64, _P, _P, _P], ct.c_int),
    "mf_gru_gates": ([_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P], ct.c_int),
    "mf_gru_sequence": ([_CFG, _I64, _I32, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _P,
                         _P, _P, _P, _P, _P, _P, _I64, _I64, _P, ct.c_uint32, ct.c_uint64, _P,
                         _I64, _P, _I64, _I32, _P, _I64, _I64, _P, _P], ct.c_int),
    "mf_stable_sum": ([_CFG, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P], ct.c_int),
    "mf_quantize_inputs_wide": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P,
                                 _P], ct.c_int),
    "mf_quantize_inputs_wide_f32": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P,
                                     _P, _P], ct.c_int),
    "mf_input_tiles_wide": ([_CFG, _P, _I64, _I64, _I64, _P, _P, _P, _P], ct.c_int),
    "mf_conv_input_tiles_wide": ([_CFG, _P, ct.POINTER(MFConvGeometry), _P, _I64, _I64, _P, _P,
                                  _P, _P, _P, _P], ct.c_int),
    "mf_quantize_weights_wide": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P,
                                  _P, _P], ct.c_int),
    "mf_quantize_weights_wide_f32": ([_CFG, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P,
                                      _P, _P, _P], ct.c_int),
    "mf_restore_wide": ([_CFG, _P, _I64, _I64, _I64, _I64, ct.c_uint32, ct.c_uint64, _P, _P],
                        ct.c_int),
    "mf_partial_wide": ([_CFG, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, ct.c_uint32, ct.c_uint64,
                         _P, _P, _P], ct.c_int),
    "mf_mm_wide": ([_CFG, _P, _P, _I64, _I64, _P, _P, _I64, _P, ct.c_uint32, ct.c_uint64, _P,
                    _I64, _P, _I64, _I32, _P, _P], ct.c_int),
    "mf_mm_totals_wide": ([_CFG, _P, _I64, _I64, _P, _I64, _P, ct.c_uint32, ct.c_uint64, _P,
                           _P, _I64, _P], ct.c_int),
    "mf_profile_kernels": ([_I32], ct.c_int),
    "mf_profile_collect": ([ct.POINTER(_I64), ct.POINTER(ct.c_double)], ct.c_int),
    "mf_mm_workspace": ([_CFG, _I64, _I64, _I64, _I32, ct.POINTER(_I64)], ct.c_int),
    "mf_mm_kernel": ([_CFG, _I64, _I64, _I64, _I32, ct.POINTER(_I32)], ct.c_int),
    "mf_resources_query": ([_CFG, _I32, _I64, _I32, ct.POINTER(MFResources)], ct.c_int),
    "mf_rng_uniform": ([_P, _I64, ct.c_uint64, ct.c_uint32, _P, _P], ct.c_int),
    "mf_rng_normal": ([_P, _I64, ct.c_uint64, ct.c_uint32, _P, _P], ct.c_int),
}


@lru_cache(None)
def library():
    """Load libmemfast_hip.so after torch, so both share one HIP runtime."""
    if not LIBRARY.is_file():
        raise BackendError(
            f"{LIBRARY} is missing; build it with `python -m memfast_amd.build_native` "
            "(memfast_amd has no CPU fallback)"
        )
    lib = ct.CDLL(str(LIBRARY))
    for name, (args, result) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = result
    if lib.mf_abi_version() != ABI_VERSION:
        raise BackendError("libmemfast_hip.so ABI version differs from memfast_amd")
    return lib


def native_source_hash():
    return library().mf_source_hash().decode()


def check(status, operation):
    if status == OK:
        return
    message = library().mf_last_error().decode(errors="replace")
    text = f"{operation} failed: {message}"
    if status == E_INVALID:
        raise ValueError(text)
    if status == E_UNSUPPORTED:
        raise NotImplementedError(text)
    if status == E_RESOURCE:
        raise ResourceError(text)
    raise BackendError(f"{text} (HIP status {status})")


def _ptr(tensor):
    return ct.c_void_p(tensor.data_ptr()) if tensor is not None else None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_get_device = getattr(torch._C, "_cuda_getDevice", None)


def _current_device():
    """torch.cuda.current_device(), without its lazy-initialisation check once the HIP
    runtime is up (every caller here already holds device tensors)."""
    if _get_device is not None and torch.cuda.is_initialized():
        return _get_device()
    return torch.cuda.current_device()


def _stream(device):
    """The current HIP stream of ``device`` as a pointer."""
    if _raw_stream is not None and isinstance(device, torch.device):
        index = device.index if device.index is not None else _current_device()
        return ct.c_void_p(_raw_stream(index))
    return ct.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class _Unchanged:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_UNCHANGED = _Unchanged()


def _on(device):
    """torch.cuda.device(device), skipped when it is already the current device."""
    if not isinstance(device, torch.device):
        return torch.cuda.device(device)
    if device.index is None or device.index == _current_device():
        return _UNCHANGED
    return torch.cuda.device(device)


def require_device(tensor):
    if not tensor.is_cuda:
        raise BackendError("memfast_amd kernels run on HIP devices only (tensor is on CPU)")


# ---------------------------------------------------------------------------
# Config -> descriptor
# ---------------------------------------------------------------------------
@lru_cache(maxsize=512)
def descriptor(config):
    """mf_config for a (hashable, frozen) Config."""
    ni = config.nonidealities
    d = MFConfig()
    d.abi_version = ABI_VERSION
    d.rows, d.cols = config.array_size
    d.read_rows = config.read_rows
    d.reads = config.reads_per_array
    d.activation_bits = config.activation_bits
    d.weight_bits = config.weight_bits
    d.weight_signed = int(config.weight_signed)
    il, wl = config.input_layout, config.weight_layout
    if len(il) > MAX_SLICES or len(wl) > MAX_SLICES:
        raise NotImplementedError("more than 32 slices")
    d.n_in, d.n_w = len(il), len(wl)
    for index, (shift, mask, factor) in enumerate(il):
        d.in_shift[index], d.in_mask[index], d.in_factor[index] = shift, mask, factor
    for index, (shift, mask, factor) in enumerate(wl):
        d.w_shift[index], d.w_mask[index], d.w_factor[index] = shift, mask, factor
    maxima = config.adc_maxima
    for index, value in enumerate(maxima):
        d.adc_max[index] = value
        d.f_alpha_over_max[index] = ni.adc_nonlinearity / value
        d.d_alpha_over_max[index] = ni.adc_nonlinearity / value
    d.precise = int(config.precise_currents)
    d.read_mode = READ_MODES[ni.read_mode]
    drift = ni.drift_factor
    d.has_write = int(ni.write_variation != 0)
    d.has_read = int(ni.read_variation != 0)
    d.has_vnoise = int(ni.voltage_variation != 0)
    d.has_nonlinear = int(ni.adc_nonlinearity != 0)
    d.has_saf = int(ni.stuck_at_low + ni.stuck_at_high != 0)
    d.has_drift = int(drift != 1.0)
    high, low, volt = config.high_conductance, config.low_conductance, config.read_voltage
    unit = config.current_unit
    # ctypes rounds Python floats to FP32 like torch rounds scalars meeting FP32 tensors.
    d.f_high, d.f_low, d.f_voltage, d.f_span = high, low, volt, high - low
    d.f_inv_unit = 1 / unit
    d.f_write, d.f_read, d.f_vnoise = ni.write_variation, ni.read_variation, ni.voltage_variation
    d.f_drift = drift
    d.f_saf_low = ni.stuck_at_low
    d.f_saf_band = ni.stuck_at_low + ni.stuck_at_high
    sigma = ni.read_variation
    d.f_out_mean = math.expm1(0.5 * sigma**2)
    d.f_out_var = math.exp(sigma**2) * math.expm1(sigma**2)
    d.f_two_pi = 2 * math.pi
    d.d_high, d.d_low, d.d_voltage, d.d_span = high, low, volt, high - low
    d.d_inv_unit = 1 / unit
    d.d_drift = drift
    d.wide = int(config.wide)
    d.bw_e = 0 if config.bw_e is None else config.bw_e
    return d


def needs_conductances(config):
    ni = config.nonidealities
    return bool(
        ni.write_variation
        or ni.stuck_at_low + ni.stuck_at_high
        or (ni.read_variation and ni.read_mode != "output")
    )


def restore_planes(config):
    ni = config.nonidealities
    if ni.read_variation and ni.read_mode == "slice_pair":
        return len(config.input_layout)
    return 1


def supported(config):
    """Raise NotImplementedError for configurations the HIP backend lacks."""
    if len(config.input_layout) > MAX_SLICES or len(config.weight_layout) > MAX_SLICES:
        raise NotImplementedError("more than 32 slices")


def _u32(codes):
    """Wide codes (values below 2^32) as the uint32 bit patterns the kernels read."""
    if codes.dtype == torch.int32:
        return codes.contiguous()
    return codes.to(torch.int64).bitwise_and(0xFFFFFFFF).to(torch.int32).contiguous()


# ---------------------------------------------------------------------------
# Programming and quantization
# ---------------------------------------------------------------------------
def _group_dims(shape, granularity):
    rows, cols = shape
    gr = rows if granularity[0] is None else min(granularity[0], rows)
    gc = cols if granularity[1] is None else min(granularity[1], cols)
    return gr, gc


STATUS_INPUT, STATUS_WEIGHT, STATUS_OUTPUT = 1, 2, 4
# mm_from_float: a group scale above the bound that keeps every FP32 output finite, so
# STATUS_OUTPUT is known only after the read (MF_STATUS_RANGE).
STATUS_RANGE = 16
# Set by a torch reduction in weight_tiles, not by a kernel: a negative weight under an
# unsigned configuration, raised after the finiteness flags as the reference orders them
# (memfast/functional.py:51-53 before memfast/quantization.py:14-18).
STATUS_NEGATIVE_WEIGHT = 8
UNSIGNED_MESSAGE = ("unsigned floating weights must be nonnegative INT values; "
                    "use map_quantized with zero_points for affine weights")


class _Scratch(ct.c_void_p):
    """A device address inside a scratch tensor, which it keeps alive until the
    launch that uses it has been queued (the caching allocator then orders any
    reuse of the memory after the launch on the same stream)."""

    __slots__ = ("owner",)


def _work_words(groups, device):
    """Group-maximum words alone (the scales go straight to the per-read table)."""
    block = torch.empty(groups, dtype=torch.int32, device=device)
    work = _Scratch(block.data_ptr())
    work.owner = block
    return work


def _group_scratch(groups, device):
    """Group-maximum words and group scales (4 bytes each, ``groups`` of both)
    in one allocation; the scales start at a 256-byte boundary."""
    offset = -(-groups // 64) * 64
    block = torch.empty(offset + groups, dtype=torch.int32, device=device)
    work, scale = _Scratch(block.data_ptr()), _Scratch(block.data_ptr() + 4 * offset)
    work.owner = scale.owner = block
    return work, scale


def status_word(device):
    """Zeroed device status word (int32) that kernels OR their MF_STATUS_* bits into."""
    return torch.zeros(1, dtype=torch.int32, device=device)


def mailbox():
    """A pinned host word for ``mm_from_float`` to publish its quantizers' status bits into."""
    return torch.zeros(1, dtype=torch.int32, pin_memory=True)


def narrow_output(output, cols, status):
    """FP32 copy [n, cols] of a wide read's FP64 output [n, >= cols] (mf_narrow_output):
    torch's cast, with a non-finite result flagged as STATUS_OUTPUT in ``status``."""
    if output.dtype != torch.float64 or output.dim() != 2 or output.stride(1) != 1:
        raise ValueError("narrow_output takes a row-major FP64 matrix")
    n = output.shape[0]
    out = torch.empty((n, cols), dtype=torch.float32, device=output.device)
    if n and cols:
        with _on(output.device):
            check(library().mf_narrow_output(_ptr(output), n, cols, output.stride(0), _ptr(out),
                                             _ptr(status), _stream(output.device)),
                  "output cast")
    return out


def status_publish(status, box):
    """Queue a copy of ``status`` into the pinned ``box`` (mf_status_publish): the bits the
    kernels queued so far set, for ``status_wait``."""
    with _on(status.device):
        check(library().mf_status_publish(_ptr(status), _ptr(box), _stream(status.device)),
              "status publish")


def status_wait(box, timeout_s=10.0):
    """The status bits ``mm_from_float`` published into ``box`` (mf_status_wait), or None
    when nothing was published within ``timeout_s`` (the caller then reads its device
    status word, which waits for the whole call)."""
    flags, published = ct.c_uint32(), _I32()
    check(library().mf_status_wait(box.data_ptr(), int(timeout_s * 1e6), ct.byref(flags),
                                   ct.byref(published)), "status wait")
    return int(flags.value) if published.value else None


def input_error(config, fixed_scale=None):
    """The reference's message for non-finite activations (memfast/quantization.py:12-13 for
    grouped scales, :124-125 for fixed scales)."""
    if fixed_scale is not None:
        return "quantized values must be finite"
    # The dtype follows the operand's own width (quantization.py:11).
    wide = config.activation_bits > 8 or config.bw_e is not None
    return f"quantized values must be finite in {torch.float64 if wide else torch.float32}"


def input_tiles(value, config, fixed_scale=None, *, status=None):
    """Codes q [N, m, R] (uint8) and per-read scales [N, m*Gr] (quantization.py:115-137).

    Without ``status`` a non-finite value raises here (quantization.py:25-26);
    with a status word the check is deferred: STATUS_INPUT is set on the device.
    """
    supported(config)
    require_device(value)
    if config.wide:
        return _input_tiles_wide(value, config, fixed_scale, status)
    n, k = value.shape
    if status is None and not torch.isfinite(value).all():
        raise ValueError(input_error(config, fixed_scale))
    x = value.to(torch.float32).contiguous()
    r = config.array_size[0]
    m = math.ceil(k / r)
    q = torch.empty((n, m, r), dtype=torch.uint8, device=value.device)
    xscale = torch.empty((n, m * config.reads_per_array), dtype=torch.float32, device=value.device)
    descr = ct.byref(descriptor(config))
    with _on(value.device):
        if fixed_scale is None:
            gr, gc = _group_dims(x.shape, config.input_quant_gran)
            groups = math.ceil(n / gr) * math.ceil(k / gc)
            if gr == 1 and gc == config.read_rows and k == m * r:
                # Groups of one read: the group grid is xscale itself.
                work, scale = _work_words(groups, value.device), _ptr(xscale)
            else:
                work, scale = _group_scratch(groups, value.device)
            check(
                library().mf_quantize_inputs(
                    descr, _ptr(x), n, k, k, gr, gc, work, scale, _ptr(q),
                    _ptr(xscale), _ptr(status), _stream(value.device),
                ),
                "input quantization",
            )
            return q, xscale
        if status is not None:
            bad = torch.isfinite(x).all().logical_not().to(torch.int32) * STATUS_INPUT
            status.bitwise_or_(bad)
        scale = fixed_scale.to(device=value.device, dtype=torch.float32).reshape(-1).contiguous()
        if scale.numel() != k:
            raise ValueError("fixed input scale must have one entry per input feature")
        check(
            library().mf_input_tiles(
                descr, _ptr(x), n, k, k, _ptr(scale), _ptr(q), _ptr(xscale), _stream(value.device),
            ),
            "input tiles",
        )
    return q, xscale


def conv_input_tiles(x, config, geometry, fixed_scale=None, *, status=None):
    """Input tiles of one convolution group's patch matrix, gathered from NCHW ``x``.

    Equals ``input_tiles(F.unfold(x, ...)[:, group block].transpose(1, 2).reshape(-1, K))``
    (memfast/nn/convolution.py:49-54) without building the patch matrix.  ``geometry``
    holds (c0, group_channels, kernel_size, stride, padding, dilation, out_size).
    Wide configurations gather from the FP64 image into uint32 codes and FP64 scales,
    as ``input_tiles`` quantizes them.  A non-finite gathered value raises here without
    ``status``, else sets STATUS_INPUT."""
    supported(config)
    require_device(x)
    wide = config.wide
    real = torch.float64 if wide else torch.float32
    c0, cg, kernel, stride, padding, dilation, out_size = geometry
    value = x.to(real).contiguous()
    n = value.shape[0]
    rows = n * out_size[0] * out_size[1]
    k = cg * kernel[0] * kernel[1]
    r = config.array_size[0]
    m = math.ceil(k / r)
    q = torch.empty((rows, m, r), dtype=torch.int32 if wide else torch.uint8, device=x.device)
    xscale = torch.empty((rows, m * config.reads_per_array), dtype=real, device=x.device)
    geom = MFConvGeometry(n, value.shape[1], value.shape[2], value.shape[3], c0, cg,
                          out_size[0], out_size[1], kernel[0], kernel[1], stride[0], stride[1],
                          padding[0], padding[1], dilation[0], dilation[1])
    own_status = status if status is not None else status_word(x.device)
    scale = work = fixed = None
    gr = gc = 0
    if fixed_scale is None:
        gr, gc = _group_dims((rows, k), config.input_quant_gran)
        grid = (math.ceil(rows / gr), math.ceil(k / gc))
        scale = torch.empty(grid, dtype=real, device=x.device)
        work = torch.empty(grid, dtype=torch.int64 if wide else torch.int32, device=x.device)
    else:
        fixed = fixed_scale.to(device=x.device, dtype=real).reshape(-1).contiguous()
        if fixed.numel() != k:
            raise ValueError("fixed input scale must have one entry per input feature")
    entry = library().mf_conv_input_tiles_wide if wide else library().mf_conv_input_tiles
    with _on(x.device):
        check(
            entry(
                ct.byref(descriptor(config)), _ptr(value), ct.byref(geom), _ptr(fixed), gr, gc,
                _ptr(work), _ptr(scale), _ptr(q), _ptr(xscale), _ptr(own_status),
                _stream(x.device),
            ),
            "conv input tiles",
        )
    if status is None and int(own_status.item()) & STATUS_INPUT:
        raise ValueError(input_error(config, fixed_scale))
    return q, xscale


def _input_tiles_wide(value, config, fixed_scale, status):
    """Wide input tiles: q [N, m, R] uint32 codes (int32 storage), FP64 scales [N, m*Gr]."""
    n, k = value.shape
    # FP32 activations are widened inside the dynamic quantizer as it reads them.
    fp32 = value.dtype == torch.float32 and fixed_scale is None
    x = value.contiguous() if fp32 else value.to(torch.float64).contiguous()
    if status is None and not torch.isfinite(x).all():
        raise ValueError(input_error(config, fixed_scale))
    r = config.array_size[0]
    m = math.ceil(k / r)
    q = torch.empty((n, m, r), dtype=torch.int32, device=value.device)
    xscale = torch.empty((n, m * config.reads_per_array), dtype=torch.float64, device=value.device)
    descr = ct.byref(descriptor(config))
    with _on(value.device):
        if fixed_scale is None:
            gr, gc = _group_dims(x.shape, config.input_quant_gran)
            grid = (math.ceil(n / gr), math.ceil(k / gc))
            scale = torch.empty(grid, dtype=torch.float64, device=value.device)
            work = torch.empty(grid, dtype=torch.int64, device=value.device)
            quantize = (library().mf_quantize_inputs_wide_f32 if fp32
                        else library().mf_quantize_inputs_wide)
            check(
                quantize(
                    descr, _ptr(x), n, k, k, gr, gc, _ptr(work), _ptr(scale), _ptr(q),
                    _ptr(xscale), _ptr(status), _stream(value.device),
                ),
                "wide input quantization",
            )
            return q, xscale
        if status is not None:
            bad = torch.isfinite(x).all().logical_not().to(torch.int32) * STATUS_INPUT
            status.bitwise_or_(bad)
        scale = fixed_scale.to(device=value.device, dtype=torch.float64).reshape(-1).contiguous()
        if scale.numel() != k:
            raise ValueError("fixed input scale must have one entry per input feature")
        check(
            library().mf_input_tiles_wide(
                descr, _ptr(x), n, k, k, _ptr(scale), _ptr(q), _ptr(xscale), _stream(value.device),
            ),
            "wide input tiles",
        )
    return q, xscale


def _check_unsigned(b, config, status):
    """Unsigned weights must be nonnegative (memfast/quantization.py:14-18): raised here, or
    with a status word flagged as STATUS_NEGATIVE_WEIGHT for the caller's one status read."""
    if config.weight_signed:
        return
    if status is None:
        if (b < 0).any():
            raise ValueError(UNSIGNED_MESSAGE)
    else:
        status.bitwise_or_((b < 0).any().to(torch.int32) * STATUS_NEGATIVE_WEIGHT)


def weight_tiles(weight, config, *, transposed=True, status=None):
    """PyTorch [O,K] weights -> packed [m,p,R,C], packed_t [p*C, m*R], scales [m*Gr,p,C].

    Follows quantization.py:82-112 (weights are quantized in physical [K,O]
    coordinates).  ``packed_t`` is the column-major copy read by the MFMA kernel.
    Without ``status`` a non-finite weight (or, for unsigned weights, a negative one)
    raises here; with a status word the checks are deferred (STATUS_WEIGHT,
    STATUS_NEGATIVE_WEIGHT).
    """
    supported(config)
    require_device(weight)
    if config.wide:
        return _weight_tiles_wide(weight, config, status)
    o, k = weight.shape
    b = weight.detach().T.to(torch.float32).contiguous()  # [K, O]
    if status is None and not torch.isfinite(b).all():
        raise ValueError("quantized values must be finite in torch.float32")
    _check_unsigned(b, config, status)
    r, c = config.array_size
    m, p = math.ceil(k / r), math.ceil(o / c)
    device = b.device
    gr, gc = _group_dims(b.shape, config.weight_quant_gran)
    groups = math.ceil(k / gr) * math.ceil(o / gc)
    packed = torch.empty((m, p, r, c), dtype=torch.uint8, device=device)
    packed_t = torch.empty((p * c, m * r), dtype=torch.uint8, device=device) if transposed else None
    wscale = torch.empty((m * config.reads_per_array, p, c), dtype=torch.float32, device=device)
    if gc == 1 and gr == config.read_rows and k == m * r and o == p * c:
        # Groups of one read of one column: the group grid is wscale itself.
        work, scale = _work_words(groups, device), _ptr(wscale)
    else:
        work, scale = _group_scratch(groups, device)
    with _on(device):
        check(
            library().mf_quantize_weights(
                ct.byref(descriptor(config)), _ptr(b), k, o, o, gr, gc, work, scale,
                _ptr(packed), _ptr(packed_t), _ptr(wscale), _ptr(status), _stream(device),
            ),
            "weight quantization",
        )
    return packed, packed_t, wscale


def _weight_tiles_wide(weight, config, status):
    """Wide programming: packed int64 [m,p,R,C], its uint32 kernel copy, FP64 scales."""
    o, k = weight.shape
    # [K, O]; FP32 weights are widened inside the quantizer as it reads them.
    source = weight.detach().T
    fp32 = source.dtype == torch.float32
    b = source.contiguous() if fp32 else source.to(torch.float64).contiguous()
    if status is None and not torch.isfinite(b).all():
        # The reference quantizes an INT operand of at most 8 bits in FP32 (per operand).
        narrow = config.weight_bits <= 8 and config.bw_e is None
        raise ValueError("quantized values must be finite in "
                         f"torch.float{32 if narrow else 64}")
    _check_unsigned(b, config, status)
    r, c = config.array_size
    m, p = math.ceil(k / r), math.ceil(o / c)
    device = b.device
    gr, gc = _group_dims(b.shape, config.weight_quant_gran)
    grid = (math.ceil(k / gr), math.ceil(o / gc))
    scale = torch.empty(grid, dtype=torch.float64, device=device)
    work = torch.empty(grid, dtype=torch.int64, device=device)
    packed = torch.empty((m, p, r, c), dtype=torch.int64, device=device)
    packed32 = torch.empty((m, p, r, c), dtype=torch.int32, device=device)
    wscale = torch.empty((m * config.reads_per_array, p, c), dtype=torch.float64, device=device)
    with _on(device):
        check(
            (library().mf_quantize_weights_wide_f32 if fp32
             else library().mf_quantize_weights_wide)(
                ct.byref(descriptor(config)), _ptr(b), k, o, o, gr, gc, _ptr(work), _ptr(scale),
                _ptr(packed), _ptr(packed32), _ptr(wscale), _ptr(status), _stream(device),
            ),
            "wide weight quantization",
        )
    if max(config.activation_bits, config.weight_bits) <= 8:
        packed = packed.to(torch.uint8)   # BFP at 8 bits keeps the reference's u8 buffer
    return packed, packed32, wscale


def kernel_codes(packed, config):
    """The read kernels' copy of programmed codes: column-major u8 codes (MFMA
    kernels, narrow) or uint32 codes in the packed layout (wide)."""
    if config.wide:
        return _u32(packed)
    return transpose_packed(packed, config)


def transpose_packed(packed, config):
    """packed [m,p,R,C] -> packed_t [p*C, m*R] (for checkpoints and imported codes)."""
    require_device(packed)
    m, p, r, c = packed.shape
    packed_t = torch.empty((p * c, m * r), dtype=torch.uint8, device=packed.device)
    src = packed.to(torch.uint8).contiguous()
    with _on(packed.device):
        check(
            library().mf_transpose_packed(
                ct.byref(descriptor(config)), _ptr(src), m, p, _ptr(packed_t),
                _stream(packed.device),
            ),
            "transpose packed",
        )
    return packed_t


# ---------------------------------------------------------------------------
# Conductances, partial totals, fused product
# ---------------------------------------------------------------------------
def restore(packed, config, seed, event, begin, end):
    """Programmed + read conductances g [planes, m, end-begin, W, R, C]."""
    supported(config)
    require_device(packed)
    m, p, r, c = packed.shape
    planes = restore_planes(config)
    dtype = torch.float64 if config.precise_currents else torch.float32
    g = torch.empty((planes, m, end - begin, len(config.weight_layout), r, c), dtype=dtype,
                    device=packed.device)
    wide = config.wide
    src = _u32(packed) if wide else packed.to(torch.uint8).contiguous()
    entry = library().mf_restore_wide if wide else library().mf_restore
    with _on(packed.device):
        check(
            entry(ct.byref(descriptor(config)), _ptr(src), m, p, begin, end, seed, event, _ptr(g),
                  _stream(packed.device)),
            "restore",
        )
    return g


def _checked_conductance(g, config, m, width, r, c):
    """Validate an injected or restored conductance tensor [planes, m, width, W, R, C]."""
    expected = (restore_planes(config), m, width, len(config.weight_layout), r, c)
    if g.dim() == 5:
        g = g.unsqueeze(0)
    if tuple(g.shape) != expected:
        raise ValueError(f"conductance tensor must have shape {expected}, got {tuple(g.shape)}")
    require_device(g)
    return g.to(torch.float64 if config.precise_currents else torch.float32).contiguous()


def partial(q, packed, config, schedule, seed, event, begin, end, *, conductance=None,
            codes=False):
    """Integer slice totals T [N, m*Gr, end-begin, C], as memfast/cuda.py:322-373.

    FP32, or FP64 for wide configurations (as the reference returns them).

    ``conductance`` injects a [planes, m, end-begin, W, R, C] tensor in place of
    the sampled one; ``codes=True`` also returns per-pair ADC counts
    [N, m*Gr, A, W, (end-begin)*C] (int32).  ``schedule`` is accepted for
    interface compatibility; the HIP kernels choose their own tiling.
    """
    supported(config)
    require_device(q)
    n, m, r = q.shape
    p, c = packed.shape[1], config.array_size[1]
    width = end - begin
    g = conductance
    if g is None and needs_conductances(config):
        g = restore(packed, config, seed, event, begin, end)
    if g is not None:
        g = _checked_conductance(g, config, m, width, r, c)
    groups = m * config.reads_per_array
    wide = config.wide
    totals = torch.empty((n, groups, width, c), dtype=torch.float64 if wide else torch.float32,
                         device=q.device)
    counts = None
    if codes:
        counts = torch.empty(
            (n, groups, len(config.input_layout), len(config.weight_layout), width * c),
            dtype=torch.int32, device=q.device,
        )
    codes_q = _u32(q) if wide else q.contiguous()
    codes_w = _u32(packed) if wide else packed.to(torch.uint8).contiguous()
    entry = library().mf_partial_wide if wide else library().mf_partial
    with _on(q.device):
        check(
            entry(ct.byref(descriptor(config)), _ptr(codes_q), n, m, _ptr(codes_w), p, begin,
                  end, _ptr(g), seed, event, _ptr(totals), _ptr(counts), _stream(q.device)),
            "partial",
        )
    return (totals, counts) if codes else totals


REUSE_TERMS = 0x100   # MF_MM_REUSE_TERMS
SPLIT_SHIFT, TIER_SHIFT = 12, 16   # MF_MM_SPLIT_SHIFT, MF_MM_TIER_SHIFT


def variant_word(tile=0, split=0, tier=0):
    """The schedule fields of mf_mm's ``variant`` (include/memfast_hip.h): the ideal read's
    tiling (0-2), the noisy read's read split (0 automatic, 1 never, s chunks) and the wide
    read's LDS tier (0 automatic, 1-3)."""
    if not (0 <= tile <= 2 and 0 <= split <= 15 and 0 <= tier <= 3):
        raise ValueError("schedule fields out of range")
    return tile | split << SPLIT_SHIFT | tier << TIER_SHIFT


def terms_event_independent(config):
    """Whether the noisy read's sampled conductances are the same on every read event."""
    return not config.nonidealities.read_variation


def mm(q, xscale, packed, packed_t, wscale, config, seed, event, *, conductance=None, out=None,
       variant=0, status=None, workspace=None, reuse_terms=False, out_cols=None, k_rows=None):
    """Fused read + scale restore: [N, p*C] FP32, summed over reads in torch's order.

    Wide configurations: ``packed_t`` is the uint32 kernel copy of the codes
    (``kernel_codes``), scales and the output are FP64 (restore_scales).
    ``workspace`` (optional, at least ``mm_workspace_bytes``) is the MFMA
    kernels' scratch; with ``reuse_terms`` it still holds the conductance terms
    a previous call of this program sampled (honoured when they do not depend
    on the read event).  ``out_cols``/``k_rows`` (default: all) are the logical
    output columns and input rows; the MFMA kernels leave columns past
    ``out_cols`` unwritten and skip reads wholly past row ``k_rows``.
    """
    supported(config)
    require_device(q)
    n, m, r = q.shape
    p, c = packed.shape[1], config.array_size[1]
    if config.wide:
        return _mm_wide(q, xscale, packed, packed_t, wscale, config, seed, event,
                        conductance=conductance, out=out, status=status,
                        variant=variant & ~REUSE_TERMS)
    if out_cols is not None and not 1 <= out_cols <= p * c:
        raise ValueError("out_cols must be in [1, p*C]")
    if k_rows is not None and not 1 <= k_rows <= m * r:
        raise ValueError("k_rows must be in [1, m*R]")
    g = conductance
    kernel = mm_kernel(config, n, m, p) if g is None and packed_t is not None else 0
    if g is None and kernel == 0 and needs_conductances(config):
        g = restore(packed, config, seed, event, 0, p)
    if g is not None:
        g = _checked_conductance(g, config, m, p, r, c)
        packed_t = None
    if out is None:
        out = torch.empty((n, p * c), dtype=torch.float32, device=q.device)
    if packed_t is not None and kernel:
        size = mm_workspace_bytes(config, n, m, p, variant & ~REUSE_TERMS)
        if workspace is None:
            workspace = torch.empty(max(1, size), dtype=torch.uint8, device=q.device)
            reuse_terms = False
        elif workspace.numel() < size or workspace.device != q.device:
            raise ValueError(f"mm workspace needs {size} bytes on {q.device}")
        if reuse_terms and kernel == 2:
            variant |= REUSE_TERMS
    else:
        workspace = None
    # Converted operands stay referenced until the launch is queued (a freed
    # temporary could be handed to the next conversion by the caching allocator).
    q, xscale = q.contiguous(), xscale.contiguous()
    packed, wscale = packed.contiguous(), wscale.contiguous()
    with _on(q.device):
        check(
            library().mf_mm(
                ct.byref(descriptor(config)), _ptr(q), _ptr(xscale), n,
                m, _ptr(packed), _ptr(packed_t), _ptr(wscale), p,
                p * c if out_cols is None else out_cols, m * r if k_rows is None else k_rows,
                _ptr(g), seed, event, _ptr(out), out.stride(0), _ptr(workspace),
                0 if workspace is None else workspace.numel(), variant, _ptr(status),
                _stream(q.device),
            ),
            "mm",
        )
    return out


def _mm_wide(q, xscale, packed, codes, wscale, config, seed, event, *, conductance, out, status,
             variant=0):
    n, m, r = q.shape
    p, c = packed.shape[1], config.array_size[1]
    codes = _u32(packed) if codes is None else _u32(codes)
    g = conductance
    workspace = None
    if g is None and mm_kernel(config, n, m, p) == 3:
        # The wide MFMA read samples conductances itself.
        workspace = _workspace(config, n, m, p, q.device, variant)
    elif g is None and needs_conductances(config):
        g = restore(codes, config, seed, event, 0, p)
    if g is not None:
        g = _checked_conductance(g, config, m, p, r, c)
    if out is None:
        out = torch.empty((n, p * c), dtype=torch.float64, device=q.device)
    q = _u32(q)
    xscale = xscale.to(torch.float64).contiguous()
    wscale = wscale.to(torch.float64).contiguous()
    with _on(q.device):
        check(
            library().mf_mm_wide(
                ct.byref(descriptor(config)), _ptr(q),
                _ptr(xscale), n, m, _ptr(codes),
                _ptr(wscale), p, _ptr(g), seed, event, _ptr(out),
                out.stride(0), _ptr(workspace), 0 if workspace is None else workspace.numel(),
                variant, _ptr(status), _stream(q.device),
            ),
            "mm",
        )
    return out


@lru_cache(maxsize=4096)
def mm_workspace_bytes(config, n, m, p, variant=0):
    """Bytes of MFMA-kernel scratch ``mm`` uses for this shape and schedule (``variant``'s
    fields; 0 for the general kernel)."""
    size = ct.c_int64()
    check(library().mf_mm_workspace(ct.byref(descriptor(config)), n, m, p, variant,
                                    ct.byref(size)), "workspace size")
    return size.value


def _workspace(config, n, m, p, device, variant=0):
    """Device scratch for the MFMA reads (mf_mm_workspace bytes, 256-byte aligned)."""
    return torch.empty(max(1, mm_workspace_bytes(config, n, m, p, variant)), dtype=torch.uint8,
                       device=device)


def bias_add(out, bias, status=None):
    """out += bias in place (FP32 [N, O], row stride out.stride(0)); a non-finite sum sets
    STATUS_OUTPUT in ``status``."""
    require_device(out)
    if out.dtype != torch.float32 or out.stride(1) != 1 or bias.shape != (out.shape[1],):
        raise ValueError("bias_add takes an FP32 row-major output and a matching bias")
    bias = bias.to(device=out.device, dtype=torch.float32).contiguous()
    with _on(out.device):
        check(library().mf_bias_add(_ptr(out), out.shape[0], out.shape[1], out.stride(0),
                                    _ptr(bias), _ptr(status), _stream(out.device)), "bias add")
    return out


def gru_gates(inputs, hidden, hx):
    """PyTorch's GRU gate equations over one step's projections (FP32 [N, 3H] each,
    hx [N, H]) in one kernel; the same FP32 roundings as the separate elementwise ops."""
    require_device(inputs)
    n, width = hx.shape
    for t, cols in ((inputs, 3 * width), (hidden, 3 * width), (hx, width)):
        if (t.dtype != torch.float32 or t.ndim != 2 or t.shape != (n, cols) or t.stride(1) != 1
                or t.device != inputs.device):
            raise ValueError("gru_gates takes FP32 row-major [N, 3H], [N, 3H] and [N, H]")
    out = torch.empty((n, width), dtype=torch.float32, device=inputs.device)
    with _on(inputs.device):
        check(library().mf_gru_gates(_ptr(inputs), inputs.stride(0), _ptr(hidden), hidden.stride(0),
                                     _ptr(hx), hx.stride(0), _ptr(out), width, n, width,
                                     _stream(inputs.device)), "GRU gates")
    return out


def gru_sequence(config, projected, h0, packed, packed_t, wscale, bias, seed, event, *, reverse,
                 status, workspace, reuse_terms=False):
    """One GRU direction's hidden reads and gates (``mf_gru_sequence``): ``projected``
    [T, B, 3H] FP32 input projections, ``h0`` [B, H] FP32; the hidden program's packed
    codes, kernel codes ``packed_t``, read scales ``wscale`` [G, p*C], FP32 ``bias`` [3H]
    or None and ``seed``; step i reads at event ``event + i``.  Returns the states
    [T, B, H] in time order.  Non-finite values set bits of ``status``, which is not read."""
    supported(config)
    require_device(projected)
    if config.wide:
        raise BackendError("the native GRU sequence covers narrow configurations")
    steps, batch, three = projected.shape
    width = h0.shape[1]
    r, c = config.array_size
    m, p = math.ceil(width / r), packed.shape[1]
    shapes_ok = (three == 3 * width and tuple(h0.shape) == (batch, width)
                 and projected.dtype == h0.dtype == wscale.dtype == torch.float32
                 and projected.is_contiguous() and h0.stride(1) == 1 and packed.shape[0] == m
                 and (bias is None or (bias.dtype == torch.float32 and bias.is_contiguous()
                                       and tuple(bias.shape) == (3 * width,))))
    if not shapes_ok:
        raise ValueError("gru_sequence takes FP32 [T, B, 3H] projections, [B, H] states and a "
                         "matching hidden program")
    size = mm_workspace_bytes(config, batch, m, p, 0)
    if workspace.numel() < size or workspace.device != projected.device:
        raise ValueError(f"gru_sequence workspace needs {size} bytes on {projected.device}")
    device = projected.device
    q = torch.empty((batch, m, r), dtype=torch.uint8, device=device)
    xscale = torch.empty((batch, m * config.reads_per_array), dtype=torch.float32, device=device)
    gr, gc = _group_dims((batch, width), config.input_quant_gran)
    groups = math.ceil(batch / gr) * math.ceil(width / gc)
    if gr == 1 and gc == config.read_rows and width == m * r:
        work, scale = _work_words(groups, device), _ptr(xscale)
    else:
        work, scale = _group_scratch(groups, device)
    hidden = torch.empty((batch, p * c), dtype=torch.float32, device=device)
    out = torch.empty((steps, batch, width), dtype=torch.float32, device=device)
    wscale = wscale.contiguous()
    with _on(device):
        check(
            library().mf_gru_sequence(
                ct.byref(descriptor(config)), steps, int(reverse), batch, width, _ptr(projected),
                batch * three, three, _ptr(h0), h0.stride(0), gr, gc, work, scale, _ptr(q),
                _ptr(xscale), _ptr(packed), _ptr(packed_t), _ptr(wscale), m, p, _ptr(bias), seed,
                event, _ptr(hidden), p * c, _ptr(workspace), workspace.numel(),
                REUSE_TERMS if reuse_terms else 0, _ptr(out), batch * width, width, _ptr(status),
                _stream(device),
            ),
            "GRU sequence",
        )
    return out


def stable_sum(totals, xscale, wscale, config, col0, out):
    """FP64 overflow-safe restore + read sum of one chunk into ``out`` [N, ldo] (FP64).

    totals [N, G, width, C] from ``partial``; xscale [N, G]; wscale [G, p*C].
    Same values and order as restore_scales(...).sum(1) on the CPU
    (memfast/simulator.py:57-66, :578-585).
    """
    require_device(totals)
    n, groups, width, c = totals.shape
    if out.dtype != torch.float64 or out.stride(1) != 1:
        raise ValueError("stable sums go to a row-major FP64 output")
    totals = totals.to(torch.float32).contiguous()
    xscale = xscale.to(torch.float32).contiguous()
    wscale = wscale.to(torch.float32).contiguous()
    with _on(totals.device):
        check(
            library().mf_stable_sum(
                ct.byref(descriptor(config)), _ptr(totals), n, groups, width, _ptr(xscale),
                _ptr(wscale), wscale.shape[1], col0, _ptr(out), out.stride(0),
                _stream(totals.device),
            ),
            "stable sum",
        )
    return out


def profile_kernels(enable):
    """Start (True) or stop recording HIP events around mf_mm's read kernel."""
    check(library().mf_profile_kernels(int(bool(enable))), "profile")


def collect_kernel_times():
    """(launches, total milliseconds) of the read kernels recorded since the last call."""
    launches, ms = ct.c_int64(), ct.c_double()
    check(library().mf_profile_collect(ct.byref(launches), ct.byref(ms)), "profile collect")
    return launches.value, ms.value


def mm_totals(q, packed_t, config, seed, event, *, conductance=None):
    """Slice totals T [N, m*Gr, p, C] (FP32) from the noisy-device MFMA kernel.

    Same values as ``partial(q, packed, config, None, seed, event, 0, p)``
    (memfast/cuda.py:322-373) up to ADC rounding-boundary flips; for parity
    tests of the kernel ``mm`` uses with noisy devices.  ``conductance``
    injects FP32 conductances [m, p, W, R, C] (one plane).
    """
    supported(config)
    require_device(q)
    n, m, r = q.shape
    c = config.array_size[1]
    p = packed_t.shape[0] // c
    g = None
    if conductance is not None:
        g = conductance.to(device=q.device, dtype=torch.float32).contiguous()
        if tuple(g.shape) != (m, p, len(config.weight_layout), r, c):
            raise ValueError("injected conductances must be [m, p, W, R, C]")
    workspace = _workspace(config, n, m, p, q.device)
    groups = m * config.reads_per_array
    totals = torch.empty((n, groups, p, c), dtype=torch.float32, device=q.device)
    q, packed_t = q.contiguous(), packed_t.contiguous()
    with _on(q.device):
        check(
            library().mf_mm_totals(
                ct.byref(descriptor(config)), _ptr(q), n, m,
                _ptr(packed_t), p, _ptr(g), seed, event, _ptr(totals),
                _ptr(workspace), workspace.numel(), _stream(q.device),
            ),
            "mm totals",
        )
    return totals


def mm_totals_wide(q, packed, config, seed, event, *, conductance=None):
    """Slice totals T [N, m*Gr, p, C] (FP64) from the wide noisy-device MFMA kernel.

    Same values as ``partial(q, packed, config, None, seed, event, 0, p)`` for a
    wide configuration, up to ADC rounding-boundary flips; for parity tests.
    ``packed`` is the [m, p, R, C] program (int64 or uint32 codes);
    ``conductance`` injects FP32 conductances [m, p, W, R, C].
    """
    supported(config)
    require_device(q)
    n, m, r = q.shape
    p, c = packed.shape[1], config.array_size[1]
    g = None
    if conductance is not None:
        g = conductance.to(device=q.device, dtype=torch.float32).contiguous()
        if tuple(g.shape) != (m, p, len(config.weight_layout), r, c):
            raise ValueError("injected conductances must be [m, p, W, R, C]")
    workspace = _workspace(config, n, m, p, q.device)
    groups = m * config.reads_per_array
    totals = torch.empty((n, groups, p, c), dtype=torch.float64, device=q.device)
    q, packed = _u32(q), _u32(packed)
    with _on(q.device):
        check(
            library().mf_mm_totals_wide(
                ct.byref(descriptor(config)), _ptr(q), n, m, _ptr(packed), p, _ptr(g),
                seed, event, _ptr(totals), _ptr(workspace), workspace.numel(), _stream(q.device),
            ),
            "mm totals",
        )
    return totals


@lru_cache(maxsize=4096)
def from_float_applies(config, n, k, o):
    """Whether ``mm_from_float`` can take an [n, k] @ [k, o] product of this configuration
    (the checks mf_mm_from_float repeats, short of buffer alignment): ideal devices on the
    MFMA read, 32 rows per read, groups of one read on both sides, whole arrays."""
    if config.wide or config.read_rows != 32:
        return False
    r, c = config.array_size
    m, p = math.ceil(k / r), math.ceil(o / c)
    return (r % 128 == 0 and c % 64 == 0 and k == m * r and o == p * c
            and _group_dims((n, k), config.input_quant_gran) == (1, 32)
            and _group_dims((k, o), config.weight_quant_gran) == (32, 1)
            and mm_kernel(config, n, m, p) == 1)


def mm_from_float(x, b, config, *, status=None, variant=0, workspace=None, scratch=None,
                  mailbox=None):
    """``x [N, K] @ b [K, O]`` from floating operands in two launches (mf_mm_from_float):
    (q, xscale, (packed, packed_t, wscale), out), exactly what ``input_tiles``,
    ``weight_tiles(b.T)`` and ``mm`` return, or None where the fused route does not apply
    (nothing is launched then).  ``workspace`` (optional, ``mm_workspace_bytes``) receives
    the digit masks as ``mm`` would.  ``scratch`` (optional) is a (q, xscale, workspace)
    triple of earlier results to write again, whose earlier readers are queued on the current
    stream.  ``mailbox`` (optional, from ``mailbox()``, zeroed by the caller) receives the
    quantizers' status bits when the read starts (``status_wait``)."""
    require_device(x)
    n, k = x.shape
    o = b.shape[1]
    device = x.device
    xf = x if x.dtype == torch.float32 and x.is_contiguous() else x.float().contiguous()
    bf = b if b.dtype == torch.float32 and b.is_contiguous() else b.detach().float().contiguous()
    r, c = config.array_size
    m, p = (k + r - 1) // r, (o + c - 1) // c
    gr_x, gc_x = _group_dims((n, k), config.input_quant_gran)
    gr_w, gc_w = _group_dims((k, o), config.weight_quant_gran)
    reads = m * config.reads_per_array
    if scratch is not None:
        q, xscale, workspace = scratch
    else:
        q = torch.empty((n, m, r), dtype=torch.uint8, device=device)
        xscale = torch.empty((n, reads), dtype=torch.float32, device=device)
        if workspace is None:
            workspace = _workspace(config, n, m, p, device, variant)
    packed = torch.empty((m, p, r, c), dtype=torch.uint8, device=device)
    packed_t = torch.empty((p * c, m * r), dtype=torch.uint8, device=device)
    wscale = torch.empty((reads, p, c), dtype=torch.float32, device=device)
    out = torch.empty((n, p * c), dtype=torch.float32, device=device)
    with _on(device):
        code = library().mf_mm_from_float(
            ct.byref(descriptor(config)), xf.data_ptr(), n, k, k, bf.data_ptr(), o, o, gr_x,
            gc_x, gr_w, gc_w, q.data_ptr(), xscale.data_ptr(), packed.data_ptr(),
            packed_t.data_ptr(), wscale.data_ptr(), out.data_ptr(), p * c, workspace.data_ptr(),
            workspace.numel(), variant, _ptr(status), _ptr(mailbox), _stream(device))
    if code == E_UNSUPPORTED:
        return None
    check(code, "quantization and read")
    return q, xscale, (packed, packed_t, wscale), out


@lru_cache(maxsize=4096)
def mm_kernel(config, n, m, p, has_packed_t=True):
    """0: general kernel, 1: ideal-device MFMA, 2: noisy-device MFMA, 3: noisy-device MFMA for
    wide codes (what ``mm`` launches; a function of its arguments, cached).

    The kernels other than the general one read ``kernel_codes`` of the program."""
    out = ct.c_int32()
    check(library().mf_mm_kernel(ct.byref(descriptor(config)), n, m, p, int(has_packed_t),
                                 ct.byref(out)), "kernel selection")
    return out.value


# ---------------------------------------------------------------------------
# RNG (parity tests)
# ---------------------------------------------------------------------------
def rng(address, seed, stream, kind="uniform"):
    require_device(address)
    addr = address.to(torch.int64).contiguous()
    out = torch.empty(addr.shape, dtype=torch.float32, device=addr.device)
    fn = library().mf_rng_uniform if kind == "uniform" else library().mf_rng_normal
    with _on(addr.device):
        check(fn(_ptr(addr), addr.numel(), int(seed) & (2**64 - 1), stream, _ptr(out),
                 _stream(addr.device)), f"rng {kind}")
    return out


# ---------------------------------------------------------------------------
# Compatibility surface of memfast/cuda.py
# ---------------------------------------------------------------------------
class Program:
    """Resource view of the kernels (replaces the NVRTC Program, cuda.py:130-310)."""

    def __init__(self, config, vectors, columns):
        self.config = config
        self.vectors = vectors
        self.columns = columns

    def resources(self, config, vectors, columns, workers, kernel=None, variant=0, batch=0):
        """Resources of the instance of read kernel ``kernel`` (mf_mm_kernel's id; by default
        the ideal MFMA read for ideal devices, else the general one) that mf_mm launches for
        ``batch`` input vectors (0: a batch above 32) under the schedule word ``variant``
        (variant_word).  ``vectors``, ``columns`` and ``workers`` are the reference's launch
        keys, which the gfx950 kernels do not use."""
        info = MFResources()
        if kernel is None:
            kernel = 1 if config.nonidealities.ideal else 0
        check(library().mf_resources_query(ct.byref(descriptor(config)), kernel, batch,
                                           variant, ct.byref(info)), "resources")
        return dict(threads=info.threads, shared=info.shared_bytes, local_bytes=info.local_bytes,
                    registers=info.registers)


@lru_cache(maxsize=256)
def program(config, vectors, columns, device):
    with _on(device):
        torch.empty(0, device=device)
        return Program(config, vectors, columns)


def identity(device):
    """Hardware identity hashed into the tuning-cache key."""
    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    info = MFIdentity()
    check(library().mf_device_identity(index, ct.byref(info)), "device identity")
    return dict(
        name=info.name.decode(),
        arch=info.arch.decode(),
        compute_units=info.compute_units,
        memory=info.memory_bytes,
        driver=info.driver_version,
        runtime=info.runtime_version,
        torch=torch.__version__,
        hip=torch.version.hip,
        kernels=native_source_hash(),
    )


__all__ = [
    "ResourceError", "BackendError", "cache_root", "atomic_write", "partial", "program",
    "identity", "mm", "restore", "input_tiles", "weight_tiles", "transpose_packed",
]
