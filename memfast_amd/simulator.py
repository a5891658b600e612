"""Programming, reading, read events and the functional API's program cache.

Drop-in for the reference's memfast/simulator.py.  ``Simulator`` and ``AnalogMatrix``
keep their constructor arguments, buffers, checkpoint state, read-event bookkeeping and
error behaviour.  Reading goes to the gfx950 kernels of libmemfast_hip.so
(memfast_amd/hip.py); there is no CPU execution path.

A read (``AnalogMatrix._execute``, memfast/simulator.py:561-616 in the reference) is
one fused launch: every array tile is read, every slice pair converted, the scales
restored and the reads summed in torch's CPU order, and only [N, p*C] is written.
Errors the reference finds with host-side scans (non-finite inputs, a non-finite FP32
result that needs the FP64 retry) are flagged in a device status word that is read
once per call, before the read event advances.

Tuned mode lives in memfast_amd/tuning.py, checkpoint validation in
memfast_amd/checkpoint.py.
"""

import hashlib
import math
import weakref
from dataclasses import asdict
from functools import lru_cache
from pathlib import Path
from typing import NamedTuple

import torch
from torch import nn

from . import checkpoint, hip, host_order, tuning
from .config import Config
from .quantization import (_signed, check_read_scales, expanded_parameter, pack_weight,
                           read_starts, row_reads)
from .tuning import default_schedule, schedule_grid

_CODE_DTYPES = (torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64)
_EVENT_LIMIT = 1 << 63
# _execute_checked's `finite` for an output that the scales bound below FLT_MAX / 2.
_BOUNDED = "bounded"


def source_hash():
    """Fingerprint of the Python sources and the compiled kernel sources."""
    root = Path(__file__).parent
    digest = hashlib.sha256()
    for path in sorted(root.rglob("*.py")):
        digest.update(path.relative_to(root).as_posix().encode())
        digest.update(path.read_bytes())
    digest.update(hip.native_source_hash().encode())
    return digest.hexdigest()


def restore_scales(value, input_scale, weight_scale):
    """value * input_scale * weight_scale in FP64 without intermediate overflow
    (memfast/simulator.py:57-66): mantissas multiply, exponents add, and the product is
    rebuilt with two ldexp steps so that an exponent beyond the FP64 range saturates only
    when the result itself does."""
    parts = [torch.frexp(t.double()) for t in (value, input_scale, weight_scale)]
    mantissa = parts[0][0] * parts[1][0] * parts[2][0]
    exponent = parts[0][1] + parts[1][1] + parts[2][1]
    head = exponent.clamp(-1022, 1023)
    rebuilt = torch.ldexp(torch.ldexp(mantissa, head), exponent - head)
    return torch.where(mantissa == 0, torch.zeros_like(rebuilt), rebuilt)


def _hip_device(device):
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError(
            "memfast_amd executes on HIP (MI355X) devices only; "
            f"device {device} is not supported (no CPU execution path)"
        )
    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device is available")
    index = torch.cuda.current_device() if device.index is None else device.index
    return torch.device("cuda", index)


@lru_cache(maxsize=4096)
def _name_tag(name):
    """32-bit seed tag of a matrix name (first four bytes of its SHA-256, little-endian;
    memfast/simulator.py:428-429)."""
    return int.from_bytes(hashlib.sha256(name.encode()).digest()[:4], "little")


# ---------------------------------------------------------------------------
# Functional RHS programs
# ---------------------------------------------------------------------------
class _CacheEntry(NamedTuple):
    owner: weakref.ref     # the caller's RHS tensor, held weakly
    geometry: tuple        # its shape, strides, offset, storage and dtype when programmed
    program: "AnalogMatrix"


def _geometry(tensor):
    return (tuple(tensor.shape), tuple(tensor.stride()), tensor.storage_offset(),
            tensor.data_ptr(), tensor.dtype, tensor.device, tensor.is_neg())


class _ProgramCache(dict):
    """Programs of the functional API's right-hand matrices, keyed by the caller's tensor
    (held weakly) and the RHS entry of a batched operand.

    memfast/simulator.py:133-171 with memfast/functional.py:94-126: each call reprograms
    the RHS (in-place edits need not advance a tensor's version).  A program of the same
    tensor with the same geometry, configuration and device is kept when its codes and
    scales are unchanged; a changed program of a rank-two RHS takes over the old one's
    name and read-event counter.  A RHS read through a view of the caller's tensor (a
    vector, or a batched operand) whose tensor changed geometry is a new RHS.  Entries
    drop out when their tensor is freed."""

    def __init__(self, simulator):
        super().__init__()
        self._simulator = weakref.ref(simulator)

    def program(self, owner, index=()):
        """The program kept for ``owner`` (entry ``index``), or None."""
        entry = self.get((id(owner), index))
        return None if entry is None or entry.owner() is not owner else entry.program

    def previous(self, rhs, owner, index):
        """(program last made for this RHS or None, whether it may be kept)."""
        previous = self.program(owner, index)
        if previous is None:
            return None, False
        same_layout = self[(id(owner), index)].geometry == _geometry(owner)
        if not same_layout and owner is not rhs:
            return None, False
        simulator = self._simulator()
        keepable = (same_layout and previous.config == simulator.config
                    and previous.packed.device == simulator.device)
        return previous, keepable

    def remember(self, owner, index, program):
        key = (id(owner), index)
        cache_ref = weakref.ref(self)

        def forget(reference):
            cache = cache_ref()
            if cache is not None and key in cache and cache[key].owner is reference:
                del cache[key]

        self[key] = _CacheEntry(weakref.ref(owner, forget), _geometry(owner), program)


# Dtypes whose FP32 quantization keeps finiteness, so that the device-side check of the
# single-pass product raises exactly where a host check would.
_SINGLE_PASS = (torch.float16, torch.bfloat16, torch.float32)


class Simulator:
    """Configuration, device, and the choice of fixed defaults or a tuned schedule.

    Interface of memfast/simulator.py:69-347.  ``tuned`` selects a schedule per input
    shape, saves the winner under ``cache_dir`` and revalidates cached winners against
    the default schedule (memfast_amd/tuning.py).
    """

    def __init__(self, config=None, *, mode="default", device=None, cache_dir=None,
                 workspace_mb=1024):
        config = Config() if config is None else config
        if not isinstance(config, Config):
            raise TypeError("config must be Config")
        if mode not in ("default", "tuned"):
            raise ValueError("mode must be default or tuned")
        budget_ok = (isinstance(workspace_mb, (int, float)) and not isinstance(workspace_mb, bool)
                     and math.isfinite(workspace_mb) and workspace_mb > 0)
        if not budget_ok:
            raise ValueError("workspace_mb must be positive and finite")
        requested = "cuda" if device is None else device
        if torch.device(requested).type not in ("cpu", "cuda"):
            raise ValueError("device must be cpu or cuda")
        self.config, self.mode = config, mode
        self.device = _hip_device(requested)
        host_order.warn_if_different()
        self.cache_dir = Path(cache_dir) if cache_dir is not None else hip.cache_root() / "tuning"
        self.workspace_bytes = int(workspace_mb * 1024**2)
        self.records = []
        self._selections = {}
        self._fingerprint = None
        self._next_id = 0
        self._matrix_cache = _ProgramCache(self)
        self._status = None   # _product's device status word; replaced once it holds flags
        self._mailbox = None  # pinned host word the fused route publishes its status bits to
        self._mailbox_layers = None   # the same for layer reads (_layer_mailbox)
        self._from_float = {}   # (n, k, o) -> whether hip.mm_from_float applies
        # (shape, stream, (q, xscale, workspace)) of the last fused call, written again by the
        # next call of that shape on that stream.
        self._from_float_scratch = (None, None, None)

    def _layer_mailbox(self):
        """The pinned word that layer reads of this simulator publish their quantizers'
        status bits to (one call at a time, as the device status words)."""
        if self._mailbox_layers is None:
            self._mailbox_layers = hip.mailbox()
        return self._mailbox_layers

    def _next_name(self):
        name = f"matrix.{self._next_id}"
        self._next_id += 1
        return name

    def _relocated(self, device):
        """A simulator with this one's configuration, mode, cache and budget on ``device``."""
        return Simulator(self.config, mode=self.mode, device=device, cache_dir=self.cache_dir,
                         workspace_mb=self.workspace_bytes / 1024**2)

    # -- programming ---------------------------------------------------------
    def map(self, weight, *, bias=None, name=None, _tiles=None):
        """Low-level layer-weight adapter using PyTorch [O,K] weight layout."""
        return AnalogMatrix(weight, self, bias=bias, name=name or self._next_name(),
                            _tiles=_tiles)

    def map_quantized(self, codes, scales, *, zero_points=None, bias=None, name=None):
        """Import integer [O,K] weights as ``scales * (codes - zero_points)``."""
        return AnalogMatrix(codes, self, bias=bias, name=name or self._next_name(),
                            scales=scales, zero_points=zero_points)

    def mm(self, input, mat2, *, out=None):
        """Simulate a two-dimensional matrix product, following torch.mm."""
        if out is None and self._plain_pair(input, mat2):
            return self._product(input, mat2)[0]
        from .functional import mm

        return mm(input, mat2, simulator=self, out=out)

    def _plain_pair(self, a, b):
        """Whether ``mm(a, b)`` goes straight to the single-pass product: two non-empty
        dense matrices of one single-pass dtype on this simulator's device, with nothing
        for the general route's checks, autocast or gradients to do.  Anything else
        takes that route, which raises the reference's errors."""
        return (type(a) is torch.Tensor and type(b) is torch.Tensor
                and a.ndim == 2 and b.ndim == 2 and a.dtype == b.dtype
                and a.dtype in _SINGLE_PASS and a.layout == b.layout == torch.strided
                and a.device == b.device == self.device and self.device.type == "cuda"
                and a.shape[1] == b.shape[0] and a.numel() > 0 and b.numel() > 0
                and not (a.requires_grad or b.requires_grad)
                and not torch.is_autocast_enabled("cuda"))

    def matmul(self, input, other, *, out=None):
        """Simulate a vector, matrix, or broadcast batch product like torch.matmul."""
        from .functional import matmul

        return matmul(input, other, simulator=self, out=out)

    def report(self):
        return dict(mode=self.mode, device=str(self.device), config=asdict(self.config),
                    selections=self.records)

    def _matrix_for(self, rhs, tiles=None, *, owner=None, index=()):
        """The program of a functional RHS [K, O] read from ``owner`` (the caller's
        tensor, ``rhs`` itself by default) at batch entry ``index``
        (memfast/simulator.py:133-171).

        ``tiles`` are the RHS's freshly quantized (packed, packed_t, wscale); a keepable
        program takes them in place, which reads exactly as the reference's kept or
        renamed program would, without comparing codes on the host."""
        owner = rhs if owner is None else owner
        previous, keepable = self._matrix_cache.previous(rhs, owner, index)
        if keepable and tiles is not None and previous._accepts(tiles):
            previous._install(tiles)
            return previous
        fresh = self.map(rhs.T, name=None if previous is None else previous.name, _tiles=tiles)
        if keepable and tiles is None and previous._same_program(fresh):
            return previous
        if previous is not None:
            fresh._event = previous._event
        self._matrix_cache.remember(owner, index, fresh)
        return fresh

    def _product(self, x, rhs, *, owner=None, index=()):
        """(``x @ rhs``, the RHS program) for the functional API, with one status read
        before any state change.

        Both operands are quantized on the device and, in default mode, read at once; the
        quantizers flag non-finite values in a status word instead of host scans.  Its one
        read raises the errors of memfast/functional.py:49-53 (A before B) while this
        simulator is unchanged; only then is the RHS program committed (``_matrix_for``)
        and its read event advanced, as AnalogMatrix.forward would.  The read uses the
        name and event that the commit assigns.
        """
        config = self.config
        owner = rhs if owner is None else owner
        if self._status is None:
            self._status = hip.status_word(self.device)
        status = self._status
        try:
            flags, tiles, q, xscale, output, kept, fused, event = self._launch(
                x, rhs, owner, index, status)
        except BaseException:
            self._status = None   # kernels may still set flags in this word
            raise
        if flags:
            self._status = None
        if flags & hip.STATUS_INPUT:
            raise ValueError("A must be finite")
        if flags & hip.STATUS_WEIGHT:
            raise ValueError("B must be finite")
        if flags & hip.STATUS_NEGATIVE_WEIGHT:
            raise ValueError(hip.UNSIGNED_MESSAGE)
        if kept is not None:
            kept._install(tiles)
            program = kept
        else:
            program = self._matrix_for(rhs, tiles=tiles, owner=owner, index=index)
        if not fused:
            if program.input_scale is not None:
                q, xscale = hip.input_tiles(x.reshape(-1, x.shape[-1]), config,
                                            program.input_scale)
            return program._run(x, q, xscale), program
        output = output[:, :program.out_features].contiguous()
        finite = not flags & hip.STATUS_OUTPUT
        if not finite and not config.wide:
            output, finite = program._execute_checked(q, xscale, default_schedule(config), event,
                                                      stable=True)
        return program._finish(x, output, finite), program

    def _launch(self, x, rhs, owner, index, status):
        """The device work of ``_product`` up to its status read: both quantizers and, in
        default mode, the fused read."""
        config = self.config
        if self.mode == "default":
            fast = self._launch_from_float(x, rhs, owner, index, status)
            if fast is not None:
                return fast
        tiles = hip.weight_tiles(rhs.T, config, status=status)
        flat = x.reshape(-1, x.shape[-1])
        q, xscale = hip.input_tiles(flat, config, status=status)
        previous, keepable = self._matrix_cache.previous(rhs, owner, index)
        kept = previous if keepable and previous._accepts(tiles) else None
        name = f"matrix.{self._next_id}" if previous is None else previous.name
        event = 0 if previous is None else previous._event
        fused = (self.mode == "default" and event < _EVENT_LIMIT
                 and (kept is None or kept.input_scale is None))
        output = None
        if fused:
            k, o = rhs.shape
            p = math.ceil(o / config.array_size[1])
            packed, codes_t, wscale = tiles
            if not (config.wide or hip.mm_kernel(config, q.shape[0], q.shape[1], p)):
                codes_t = None
            # A wide read's quantizers flag STATUS_RANGE for group scales that could take the
            # output past FLT_MAX / 2; without it their bits are all the read can leave, and
            # they are published to the mailbox before the read runs.
            box = None
            if config.wide and x.dtype in (torch.float32, torch.float64):
                if self._mailbox is None:
                    self._mailbox = hip.mailbox()
                box = self._mailbox
                hip.status_publish(status, box)
            output = hip.mm(q, xscale, packed, codes_t, wscale.reshape(-1, p * config.array_size[1]),
                            config, config.seed ^ _name_tag(name), event,
                            variant=tuning.DEFAULT_VARIANT, status=status, out_cols=o, k_rows=k)
            if config.wide and x.dtype == torch.float32:
                # The cast to FP32 flags a non-finite result in the status word, so the one
                # status read below also stands for the host scan of the cast output.
                output = hip.narrow_output(output, o, status)
            if box is not None and hip.status_wait(box) == 0:
                return 0, tiles, q, xscale, output, kept, fused, event
        return int(status.item()), tiles, q, xscale, output, kept, fused, event

    def _launch_from_float(self, x, rhs, owner, index, status):
        """``_launch`` in two launches (``hip.mm_from_float``: both quantizers with the
        ideal read's digit masks, then the read) where that route applies: what the
        quantizers and the fused read produce, or None."""
        flat = x.reshape(-1, x.shape[-1])
        shape = (flat.shape[0], flat.shape[1], rhs.shape[1])
        applies = self._from_float.get(shape)
        if applies is None:
            applies = self._from_float[shape] = hip.from_float_applies(self.config, *shape)
        if not applies:
            return None
        previous, keepable = self._matrix_cache.previous(rhs, owner, index)
        event = 0 if previous is None else previous._event
        if event >= _EVENT_LIMIT or (previous is not None and previous.input_scale is not None):
            return None
        # The codes, scales and masks of the last call of this shape are written again when
        # that call ran on the current stream: its read is queued before these writes.
        last_shape, last_stream, scratch = self._from_float_scratch
        stream = hip._stream(self.device).value
        reuse = last_shape == shape and last_stream == stream
        if self._mailbox is None:
            self._mailbox = hip.mailbox()
        fused = hip.mm_from_float(flat, rhs, self.config, status=status,
                                  scratch=scratch if reuse else None, mailbox=self._mailbox)
        if fused is None:
            self._from_float[shape] = False
            return None
        q, xscale, tiles, output = fused
        if not reuse:
            workspace = hip._workspace(self.config, shape[0], q.shape[1], tiles[0].shape[1],
                                       q.device)
            self._from_float_scratch = (shape, stream, (q, xscale, workspace))
        kept = previous if keepable and previous._accepts(tiles) else None
        # The read publishes the quantizers' status bits when it starts.  Unless a scale is
        # large enough for an FP32 output to overflow, they are every bit of the call, and
        # the read finishes behind the caller's next work on the stream.
        flags = hip.status_wait(self._mailbox)
        if flags is None or flags & hip.STATUS_RANGE:
            flags = int(status.item())
        return flags, tiles, q, xscale, output, kept, True, event

    # -- tuned mode (memfast_amd/tuning.py) -------------------------------------
    def _key(self, matrix, x, grid):
        """(digest, payload) of a selection (memfast/simulator.py:195-214, grid re-keyed)."""
        if self._fingerprint is None:
            self._fingerprint = source_hash()
        return tuning.selection_key(self, matrix, x, grid, self._fingerprint)

    def _admit(self, matrix, q, schedule):
        """Resources of a schedule; ResourceError when its scratch exceeds the workspace
        budget or its kernel would spill registers."""
        c = self.config
        n, arrays, _ = q.shape
        if tuning.workspace_need(c, n, arrays, matrix.p, schedule) > self.workspace_bytes:
            raise hip.ResourceError("workspace budget")
        kernel = tuning.read_kernel(c, n, arrays, matrix.p)
        with torch.cuda.device(self.device):
            resource = hip.program(c, schedule["vectors"], schedule["columns"],
                                   self.device.index).resources(
                c, schedule["vectors"], schedule["columns"], schedule["workers"], kernel=kernel,
                variant=tuning.schedule_variant(schedule), batch=n)
        # The output-noise MFMA read at 32-row reads keeps part of its state in scratch by
        # design (three waves per SIMD with spills run faster than two without), and its
        # registers do not depend on the schedule; the policy refuses any other spill.
        n_read = c.nonidealities.read_variation > 0 and c.nonidealities.read_mode == "output"
        deliberate = kernel == 2 and n_read and c.read_rows == 32
        if resource["local_bytes"] and not deliberate:
            raise hip.ResourceError("register spill policy")
        return resource

    def _select(self, matrix, x, q, xscale, event):
        return tuning.ScheduleSearch(self, matrix, x, q, xscale, event).run()


# ---------------------------------------------------------------------------
# Program sources of an AnalogMatrix
# ---------------------------------------------------------------------------
def _from_float(weight, zero_points, simulator, tiles):
    """(packed, packed_t, weight_scale) of floating [O,K] weights, quantized on the GPU
    (memfast/quantization.py:82-112), or the caller's already quantized ``tiles``."""
    if tiles is not None:
        return tiles
    if not weight.is_floating_point():
        raise ValueError("unquantized weight must be floating")
    if zero_points is not None:
        raise ValueError("zero_points requires imported integer codes and scales")
    return hip.weight_tiles(weight.detach().to(simulator.device), simulator.config)


def _from_codes(codes, scales, zero_points, simulator):
    """(packed, weight_scale, zero_correction) of imported integer [O,K] codes with
    ``scales`` and optional ``zero_points`` (memfast/simulator.py:173-185, :380-404)."""
    config, device = simulator.config, simulator.device
    if codes.dtype not in _CODE_DTYPES:
        raise ValueError("imported weight codes must have an integer dtype")
    if config.bw_e is not None:
        raise ValueError("native INT weight import requires bw_e=None")
    signed = config.weight_signed
    low = -(1 << (config.weight_bits - 1)) if signed else 0
    high = (1 << (config.weight_bits - int(signed))) - 1
    values = codes.detach().to(device=device, dtype=torch.int64)
    if bool(values.lt(low).any()) or bool(values.gt(high).any()):
        raise ValueError("weight codes exceed configured signedness or bit width")
    dtype = torch.float64 if config.wide else torch.float32
    shape = tuple(codes.shape)
    physical_scale = expanded_parameter(scales, shape, device, dtype, "scales",
                                        positive=True).detach().T.contiguous()
    check_read_scales(physical_scale, config, "weight scale")
    packed, table = pack_weight(values.T.contiguous(), physical_scale, config)
    if zero_points is None:
        return packed, table, None
    zeros = expanded_parameter(zero_points, shape, device, dtype,
                               "zero_points").detach().T.contiguous()
    check_read_scales(zeros, config, "weight zero point")
    k = shape[1]
    first = read_starts(math.ceil(k / config.array_size[0]), config, device).clamp_max(k - 1)
    correction = -(zeros[first] * physical_scale[first])
    if not bool(torch.isfinite(correction).all()):
        raise ValueError("scaled zero points exceed the reconstruction dtype")
    return packed, table, correction


def _bias_buffer(bias, out_features, device, dtype):
    """The bias buffer in the reconstruction dtype, with the reference's checks."""
    if bias is None:
        return None
    valid = (bias.is_floating_point() and tuple(bias.shape) == (out_features,)
             and bool(torch.isfinite(bias).all()))
    if not valid:
        raise ValueError("bias must be finite and match out_features")
    stored = bias.detach().to(device=device, dtype=dtype).clone()
    if not bool(torch.isfinite(stored).all()):
        raise ValueError("bias exceeds the reconstruction dtype")
    return stored


class AnalogMatrix(nn.Module):
    """A programmed matrix: codes, scales and optional digital zero-point compensation.

    Buffers, checkpoint state and validation follow memfast/simulator.py:350-646.
    """

    def __init__(self, weight, simulator, *, bias=None, name="matrix", scales=None,
                 zero_points=None, _tiles=None):
        super().__init__()
        if weight.ndim != 2 or min(weight.shape) < 1:
            raise ValueError("weight must be a nonempty [O,K] matrix")
        if _tiles is None and not bool(torch.isfinite(weight).all()):
            raise ValueError("weights must be finite")
        self.simulator, self.config, self.name = simulator, simulator.config, name
        hip.supported(self.config)
        self.out_features, self.in_features = weight.shape
        self.p = math.ceil(self.out_features / self.config.array_size[1])
        column_codes, correction = None, None
        if scales is None:
            packed, column_codes, table = _from_float(weight, zero_points, simulator, _tiles)
        else:
            packed, table, correction = _from_codes(weight, scales, zero_points, simulator)
        dtype = torch.float64 if self.config.wide else torch.float32
        for key, tensor in (("packed", packed), ("weight_scale", table),
                            ("zero_correction", correction), ("input_scale", None),
                            ("bias", _bias_buffer(bias, self.out_features, simulator.device,
                                                  dtype))):
            self.register_buffer(key, tensor)
        self._event = 0
        self.seed = self.config.seed ^ _name_tag(name)
        self._prepared = {}          # tuned schedules by (input shape, dtype)
        self._kernel_codes = None    # (codes key, the kernels' copy of the codes)
        self._workspace = None       # noisy MFMA scratch kept across reads
        self._terms_source = None    # (kernel codes, version, seed) of the terms it holds
        if column_codes is not None:
            self._kernel_codes = (self._codes_key(), column_codes)

    # -- the kernels' copy of the codes ----------------------------------------
    def _codes_key(self, packed=None):
        packed = self.packed if packed is None else packed
        return (packed.data_ptr(), packed._version, packed.device, tuple(packed.shape))

    def _column_codes(self):
        """The kernels' copy of the codes (hip.kernel_codes), refreshed on change."""
        key = self._codes_key()
        if self._kernel_codes is None or self._kernel_codes[0] != key:
            self._kernel_codes = (key, hip.kernel_codes(self.packed, self.config))
        return self._kernel_codes[1]

    def _accepts(self, tiles):
        """Whether freshly quantized ``tiles`` can replace this program's in place."""
        packed, _, table = tiles
        own = self._buffers   # the registered buffers, without Module.__getattr__
        return (own["zero_correction"] is None and own["bias"] is None
                and own["packed"].dtype == packed.dtype and own["packed"].shape == packed.shape
                and own["weight_scale"].dtype == table.dtype
                and own["weight_scale"].shape == table.shape)

    def _install(self, tiles):
        """Take freshly quantized codes and scales of the same matrix (``_accepts``):
        the buffer table entries are replaced, as attribute assignment would."""
        packed, column_codes, table = tiles
        self._buffers["packed"], self._buffers["weight_scale"] = packed, table
        self.__dict__["_kernel_codes"] = (
            None if column_codes is None else (self._codes_key(packed), column_codes))

    def _same_program(self, other):
        return (torch.equal(self.packed, other.packed)
                and torch.equal(self.weight_scale, other.weight_scale))

    @torch.no_grad()
    def _prepare(self, weight, bias=None):
        """A new program of floating [O,K] weights (and bias) for ``_commit``, with the
        checks of programming a fresh matrix (memfast/nn/training.py:40-47); nothing of
        this matrix changes."""
        if not bool(torch.isfinite(weight).all()):
            raise ValueError("weights must be finite")
        if not weight.is_floating_point():
            raise ValueError("unquantized weight must be floating")
        packed, column_codes, table = hip.weight_tiles(weight.detach().to(self.packed.device),
                                                       self.config)
        dtype = torch.float64 if self.config.wide else torch.float32
        return packed, column_codes, table, _bias_buffer(bias, self.out_features,
                                                         self.packed.device, dtype)

    @torch.no_grad()
    def _commit(self, prepared):
        """Write a ``_prepare``d program into the existing buffers (the bias only where
        this matrix has one): buffer identities, name, seed, read count and tuned
        schedules stay."""
        packed, column_codes, table, bias = prepared
        self.packed.copy_(packed)
        self.weight_scale.copy_(table)
        if bias is not None and self.bias is not None:
            self.bias.copy_(bias)
        self._kernel_codes = None if column_codes is None else (self._codes_key(), column_codes)

    def _reprogram(self, weight, bias=None):
        self._commit(self._prepare(weight, bias))

    # -- settings ----------------------------------------------------------------
    def set_input_scale(self, scale):
        """Fix symmetric activation scales for subsequent calls; None restores dynamic scales."""
        if scale is not None:
            dtype = torch.float64 if self.config.wide else torch.float32
            fixed = expanded_parameter(scale, (1, self.in_features), self.packed.device, dtype,
                                       "input scale").detach()
            if bool((fixed <= 0).any()):
                raise ValueError("input scale must be strictly positive")
            check_read_scales(fixed.T, self.config, "input scale")
            scale = fixed.clone()
        self.input_scale = scale
        self._prepared.clear()
        return self

    def reset_read(self, event=0):
        if type(event) is not int or not 0 <= event < _EVENT_LIMIT:
            raise ValueError("event must be a nonnegative signed 64-bit integer")
        self._event = event

    @torch.no_grad()
    def update_weight(self, matrix):
        """Reprogram a right-hand [K,O] matrix without replacing this module; the read
        count restarts at zero (memfast/simulator.py:541-559)."""
        if not isinstance(matrix, torch.Tensor) or tuple(matrix.shape) != (self.in_features,
                                                                            self.out_features):
            raise ValueError("replacement matrix must have the original [K,O] shape")
        self._reprogram(matrix.T)
        self.zero_correction = None
        self._prepared.clear()
        self.reset_read()
        return self

    # -- checkpoints (memfast_amd/checkpoint.py) ---------------------------------
    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        checkpoint.check_incoming(self, state_dict, prefix)
        checkpoint.shape_optional_buffers(self, state_dict, prefix)
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        checkpoint.check_loaded(self)
        self._kernel_codes = None

    def get_extra_state(self):
        return checkpoint.extra_state(self)

    def set_extra_state(self, state):
        name, seed, event = checkpoint.check_extra_state(self, state)
        self.reset_read(event)
        self.name, self.seed = name, seed
        self._prepared.clear()

    def _apply(self, fn, recurse=True):
        """Device moves keep the programmed buffers' dtypes (memfast/simulator.py:484-493)."""
        before = {key: buffer for key, buffer in self._buffers.items() if buffer is not None}
        super()._apply(fn, recurse=recurse)
        for key, original in before.items():
            moved = self._buffers[key]
            if moved.dtype != original.dtype:
                self._buffers[key] = original.to(device=moved.device)
            if moved.device != original.device:
                self._prepared.clear()
                self._kernel_codes = None
        return self

    # -- reading -------------------------------------------------------------------
    def _execute(self, q, xscale, schedule, event, stable=False):
        """One fused read of every tile; memfast/simulator.py:561-616."""
        return self._execute_checked(q, xscale, schedule, event, stable)[0]

    def _zero_point_term(self, q, xscale, stable):
        """The digital zero-point correction [N, O] of memfast/simulator.py:587-611: each
        read's sum of signed input codes times its input scale, times the correction row
        of that read.  One FP32 matrix product, or in FP64 per C columns through
        restore_scales for wide configurations and the overflow retry."""
        config = self.config
        codes = _signed(q.reshape(q.shape[0], -1), config.activation_bits)
        reads = row_reads(codes.shape[1], config, q.device)
        sums = torch.zeros((q.shape[0], xscale.shape[1]), dtype=torch.int64, device=q.device)
        sums.index_add_(1, reads, codes)
        correction = self.zero_correction
        if not (config.wide or stable):
            return (sums.float() * xscale.float()) @ correction.float()
        width = config.array_size[1]
        term = torch.empty((q.shape[0], self.out_features), dtype=torch.float64,
                           device=q.device)
        for first in range(0, self.out_features, width):
            block = slice(first, min(first + width, self.out_features))
            term[:, block] = restore_scales(sums[:, :, None], xscale[:, :, None],
                                            correction[None, :, block]).sum(1)
        return term

    def _execute_checked(self, q, xscale, schedule, event, stable=False, status=None,
                         input_error=None, retry=True, defer=False, narrow=False):
        """(output, finite) where ``finite`` is True when the output is known finite.

        ``status`` may carry STATUS_INPUT from a deferred input quantization; the one
        status read raises ``input_error`` for it before anything else.  With ``retry``
        False, a non-finite FP32 result returns (None, False) instead of the FP64 retry
        (which changes every row's rounding).  With ``defer`` the status word is not
        read: the FP32 output returns as it is and the caller reads ``status`` later
        (``_forward_deferred``).  With ``narrow`` a wide read's FP64 output returns cast to
        FP32 on the device, its non-finite values flagged in the status word
        (hip.narrow_output), so that the caller's FP32 output needs no host scan."""
        config = self.config
        columns = self.p * config.array_size[1]
        packed = self.packed
        if not config.wide and packed.dtype != torch.uint8:
            packed = packed.to(torch.uint8)
        box = None
        if stable:
            output = self._execute_stable(q, xscale, packed, event)
        else:
            kernel = hip.mm_kernel(config, q.shape[0], q.shape[1], self.p)
            codes_t = self._column_codes() if config.wide or kernel else None
            status = hip.status_word(q.device) if status is None else status
            if not defer and self._output_bounded(q.shape[1]):
                # The quantizer's bits are the only ones this read can leave: publish them
                # now, and the read runs on behind the caller's next work.
                box = self.simulator._layer_mailbox()
                hip.status_publish(status, box)
            variant = tuning.schedule_variant(schedule)
            workspace, reuse, source = None, False, None
            if kernel == 2 and hip.terms_event_independent(config):
                workspace, reuse, source = self._terms_workspace(q.shape[0], q.shape[1], q.device,
                                                                 codes_t, variant)
            output = hip.mm(q, xscale, packed, codes_t, self.weight_scale.reshape(-1, columns),
                            config, self.seed, event, variant=variant, status=status,
                            workspace=workspace, reuse_terms=reuse,
                            out_cols=self.out_features, k_rows=self.in_features)
            if source is not None:
                self._terms_source = source
        output = output[:, :self.out_features].contiguous()
        if self.zero_correction is not None:
            output = output + self._zero_point_term(q, xscale, stable).to(output.dtype)
        # An FP32 read's bias goes through a kernel that also flags non-finite sums.
        checked_bias = (self.bias is not None and self.zero_correction is None
                        and not config.wide and not stable)
        if self.bias is not None and not checked_bias:
            output = output + self.bias
        if stable:
            return output, False
        if checked_bias:
            hip.bias_add(output, self.bias, status)
        if defer:
            return output, True
        narrowed = narrow and config.wide
        if narrowed:
            output = hip.narrow_output(output, self.out_features, status)
        if box is not None:
            flags = hip.status_wait(box)
            if flags is not None and flags & hip.STATUS_INPUT:
                raise ValueError(input_error or "quantized values must be finite")
            if flags == 0:
                return output, _BOUNDED
        flags = int(status.item())   # the one status read: deferred input check, then outputs
        if flags & hip.STATUS_INPUT:
            raise ValueError(input_error or "quantized values must be finite")
        flagged = bool(flags & hip.STATUS_OUTPUT)
        host_scan = not narrowed and (self.zero_correction is not None or
                                      (config.wide and self.bias is not None))
        finite = bool(torch.isfinite(output).all()) if host_scan else not flagged
        if finite or config.wide:
            # A wide read is already an FP64 restore; the reference's retry
            # (memfast/simulator.py:614-615) would repeat the same computation.
            return output, finite
        if not retry:
            return None, False
        return self._execute_checked(q, xscale, schedule, event, stable=True)

    def _host_max(self, name, tensor):
        """max |tensor| as a Python float, read from the device once per version of the
        tensor: the same tensor object (a replaced buffer may reuse the old one's storage)
        with the same in-place modification count."""
        cache = self.__dict__.setdefault("_host_maxima", {})
        hit = cache.get(name)
        if hit is None or hit[0]() is not tensor or hit[1] != tensor._version:
            value = float(tensor.detach().abs().max()) if tensor.numel() else 0.0
            hit = cache[name] = (weakref.ref(tensor), tensor._version, value)
        return hit[2]

    def _output_bounded(self, arrays):
        """Whether the default-mode read of fixed-scale inputs cannot leave a non-finite
        output: every read's total obeys |T| <= Config.reconstruction_bound, so with the
        largest fixed input scale xs, weight scale ws and bias b, every FP32 product, sum and
        bias add stays below G * bound * xs * ws * 1.07 + |b| (G reads), asked here to be
        below FLT_MAX / 2.  Those maxima are read once per version of their tensors."""
        if (self.simulator.mode != "default" or self.input_scale is None
                or self.config.bw_e is not None or self.zero_correction is not None):
            return False
        reads = arrays * self.config.reads_per_array
        xs = self._host_max("input_scale", self.input_scale)
        ws = self._host_max("weight_scale", self.weight_scale)
        bias = 0.0 if self.bias is None else self._host_max("bias", self.bias)
        bound = reads * self.config.reconstruction_bound * xs * ws * 1.07 + bias
        return math.isfinite(bound) and bound < torch.finfo(torch.float32).max / 2

    def _terms_workspace(self, rows, arrays, device, codes_t, variant=tuning.DEFAULT_VARIANT):
        """Workspace of the noisy MFMA read kept across calls, and whether it still holds
        this program's conductance terms (same kernel codes object and version, seed).

        Write variation, drift and stuck-at faults do not depend on the read event
        (memfast/reference.py:36-46), so those samples are identical on every read
        of a programmed matrix and need not be drawn again."""
        need = hip.mm_workspace_bytes(self.config, rows, arrays, self.p, variant)
        workspace = self._workspace
        if workspace is None or workspace.numel() < need or workspace.device != device:
            workspace = torch.empty(max(1, need), dtype=torch.uint8, device=device)
            self._workspace, self._terms_source = workspace, None
        source = (codes_t, codes_t._version, self.seed)
        held = self._terms_source
        reuse = held is not None and held[0] is codes_t and held[1:] == source[1:]
        self._terms_source = None     # set again once the call has been queued
        return workspace, reuse, source

    def _execute_stable(self, q, xscale, packed, event):
        """FP64 overflow-safe restore of the slice totals (non-finite FP32 retry).

        Chunks of two tiles as memfast/simulator.py:561-585; the restore and the read
        sum run in one kernel with torch's CPU summation order.
        """
        width = self.config.array_size[1]
        output = torch.empty((q.shape[0], self.p * width), dtype=torch.float64, device=q.device)
        wscale = self.weight_scale.reshape(-1, self.p * width)
        chunk = min(2, self.p)
        for first in range(0, self.p, chunk):
            last = min(first + chunk, self.p)
            totals = hip.partial(q, packed, self.config, None, self.seed, event, first, last)
            hip.stable_sum(totals, xscale, wscale, self.config, first * width, output)
        return output

    def _check_input(self, x):
        """Argument checks of a read (memfast/simulator.py:618-631)."""
        if x.ndim < 1 or x.shape[-1] != self.in_features or not x.is_floating_point():
            raise ValueError("input must be floating with matching in_features")
        if x.device != self.packed.device or x.device != self.simulator.device:
            raise ValueError("input and simulator must use the same device")
        if self.weight_scale.dtype != (torch.float64 if self.config.wide else torch.float32):
            raise RuntimeError("keep simulator scale buffers at their mapped dtype")

    @torch.no_grad()
    def forward(self, x):
        return self._forward(x)

    def _forward(self, x, retry=True):
        """forward(); with ``retry`` False it returns None (event unchanged) where the
        FP32 read is not finite, so that a caller batching independent rows can fall
        back to separate calls."""
        self._check_input(x)
        if x.numel() == 0:
            return x.new_empty((*x.shape[:-1], self.out_features))
        if self._event >= _EVENT_LIMIT:
            raise OverflowError("read-event counter exhausted")
        # Default mode defers the finiteness check of x to the read's status word (raised
        # before the event advances); tuned mode checks first, as its schedule search
        # runs before the read.
        status = hip.status_word(x.device) if self.simulator.mode == "default" else None
        q, xscale = hip.input_tiles(x.reshape(-1, self.in_features), self.config,
                                    self.input_scale, status=status)
        return self._run(x, q, xscale, status=status, retry=retry)

    def _deferrable(self, x, reads):
        """Whether ``reads`` reads of inputs like ``x`` can go through ``_forward_deferred``:
        default mode, narrow FP32 reads with the bias added by the checking kernel."""
        return (
            self.simulator.mode == "default" and not self.config.wide
            and self._buffers["zero_correction"] is None
            and x.dtype == torch.float32 and x.ndim == 2 and x.shape[0] > 0
            and x.shape[1] == self.in_features and x.device == self.simulator.device
            and self.weight_scale.dtype == torch.float32 and self._event + reads < _EVENT_LIMIT
        )

    def _forward_deferred(self, x, status):
        """forward() for a ``_deferrable`` input that ORs its status bits into ``status``
        and returns without reading it, so that reads can queue back to back.

        When ``status`` is still clear after the last such read, every output equals
        what forward() returns and no forward() would have raised.  When any bit is set,
        the caller restores the read count and reads again through forward(), which
        raises or retries exactly where it would have.
        """
        q, xscale = hip.input_tiles(x, self.config, self.input_scale, status=status)
        output, _ = self._execute_checked(q, xscale, default_schedule(self.config), self._event,
                                          status=status, defer=True)
        self.__dict__["_event"] = self._event + 1
        return output

    def _run(self, x, q, xscale, status=None, retry=True):
        """Read quantized inputs under the mode's schedule, then ``_finish``."""
        if self._event >= _EVENT_LIMIT:
            raise OverflowError("read-event counter exhausted")
        event = self._event
        schedule = default_schedule(self.config)
        if self.simulator.mode == "tuned":
            key = (tuple(x.shape), str(x.dtype))
            if key not in self._prepared:
                with torch.cuda.device(q.device):
                    self._prepared[key] = self.simulator._select(self, x, q, xscale, event)
            schedule = self._prepared[key]
        output, finite = self._execute_checked(
            q, xscale, schedule, event, status=status,
            input_error=hip.input_error(self.config, self.input_scale), retry=retry,
            narrow=x.dtype == torch.float32)
        return None if output is None else self._finish(x, output, finite)

    def _finish(self, x, output, finite):
        """Cast to the input dtype, check finiteness, advance the read event
        (memfast/simulator.py:632-646).  A _BOUNDED output is below FLT_MAX / 2, so it is
        finite in every input dtype with FP32's range."""
        converted = output.reshape(*x.shape[:-1], self.out_features).to(x.dtype)
        known = finite is _BOUNDED and x.dtype != torch.float16
        if not (known or (finite and output.dtype == x.dtype)) and \
                not bool(torch.isfinite(converted).all()):
            raise FloatingPointError("nonfinite analog output")
        self._event += 1
        return converted


__all__ = ["Simulator", "AnalogMatrix", "default_schedule", "schedule_grid", "restore_scales"]
