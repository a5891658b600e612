"""CPU oracle for the sliced analog matrix product (TEST INFRASTRUCTURE ONLY).

This module restates, operation for operation, the reference CPU path of
HUST-ISMD-Odyssey/MemFast 0.3.0 with torch CPU tensors.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker or the timed CPU baseline.  The product package
(``memfast_amd``) never imports it.

The operation order is kept identical to the reference wherever FP32 rounding
depends on it (voltages, conductances, ADC scaling, the (T*xs)*ws restore and
torch's own ``sum`` over reads), because bit-exact parity is judged against
that order.  Each function cites the reference lines it follows.

Pinning status (what checks each function beyond this restatement):
  * grouped_quantize / pack_weight / weight_tiles: the reference's LeNet
    float and static-INT4 checkpoints (codes, layout, padding), IEEE division
    identities, brute-force round-half-even.
  * input_tiles / read_starts: closed-form index tests, fixed-scale fixture.
  * mix / uniform / event_seed / normal: a C restatement (oracle/brute.c),
    distribution tests, and vectors written by
    tests/golden/make_reference_vectors.py.
  * partial / adc (ideal devices): C brute force of the closed form
    code = min(sum_r da*dw, max), the DFT notebook known answer.
  * partial / restored with noise: vectors written by
    tests/golden/make_reference_vectors.py (transcendentals are torch CPU).
  * execute epilogue order: torch's own CPU ``sum`` (called directly here).
  * imported_tiles / zero_point_correction (map_quantized): with ideal devices
    and an ADC that never clamps, the product equals the dequantized affine
    weights' product (tests/test_oracle.py closed form).
"""

import hashlib
import math

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# Layout helpers, computed from the raw Config fields so that this oracle
# cross-checks the product's derived properties (memfast/config.py:175-209).
# ---------------------------------------------------------------------------
def _layout(widths, bits, signed=True):
    widths = (1,) * bits if widths is None else tuple(widths)
    out, shift = [], 0
    for index, width in enumerate(reversed(widths)):
        last = index == len(widths) - 1
        out.append((shift, (1 << width) - 1, -(1 << shift) if signed and last else 1 << shift))
        shift += width
    return tuple(out)


def input_layout(cfg):
    return _layout(cfg.input_slice, cfg.activation_bits, True)


def weight_layout(cfg):
    return _layout(cfg.weight_slice, cfg.weight_bits, cfg.weight_signed)


def adc_maxima(cfg):
    count = len(weight_layout(cfg))
    bits = (cfg.adc_bits,) * count if type(cfg.adc_bits) is int else tuple(reversed(cfg.adc_bits))
    return tuple((1 << b) - 1 for b in bits)


def read_rows(cfg):
    return cfg.array_size[0] if cfg.rows_per_read is None else cfg.rows_per_read


def reads_per_array(cfg):
    return math.ceil(cfg.array_size[0] / read_rows(cfg))


def is_wide(cfg):
    return max(cfg.activation_bits, cfg.weight_bits) > 8 or cfg.bw_e is not None


def precise_currents(cfg):
    widest = max(e[1] for e in (*input_layout(cfg), *weight_layout(cfg)))
    h, lo, v = cfg.high_conductance, cfg.low_conductance, cfg.read_voltage
    return (
        widest > 255
        or h - lo < h * 1e-4
        or h * v * read_rows(cfg) > 8e37
        or min(lo, v) < 1e-18
        or max(h, v) > 1e18
    )


def current_unit(cfg):
    return (cfg.high_conductance - cfg.low_conductance) * cfg.read_voltage


def drift_factor(cfg):
    ni = cfg.nonidealities
    return (1 + ni.drift_time / ni.drift_reference_time) ** (-ni.drift_coefficient)


def name_seed(cfg_seed, name):
    """Per-matrix sampling seed (memfast/simulator.py:428-429)."""
    tag = int.from_bytes(hashlib.sha256(name.encode()).digest()[:4], "little")
    return cfg_seed ^ tag


# ---------------------------------------------------------------------------
# Counter-based RNG (memfast/random.py:8-33), int64 tensors holding u32 words.
# ---------------------------------------------------------------------------
def mix(x):
    x = x & 0xFFFFFFFF
    x = ((x ^ (x >> 16)) * 0x7FEB352D) & 0xFFFFFFFF
    x = ((x ^ (x >> 15)) * 0x846CA68B) & 0xFFFFFFFF
    return x ^ (x >> 16)


def mix_int(x):
    """Python-int version of ``mix`` for scalar keys."""
    x &= 0xFFFFFFFF
    x = ((x ^ (x >> 16)) * 0x7FEB352D) & 0xFFFFFFFF
    x = ((x ^ (x >> 15)) * 0x846CA68B) & 0xFFFFFFFF
    return x ^ (x >> 16)


def uniform(address, seed, stream):
    """24-bit uniform in (0,1) keyed by (address, seed, stream); random.py:15-23."""
    key = mix_int((int(seed) ^ (int(stream) * 0x9E3779B9)) & 0xFFFFFFFF)
    high = address >> 32
    folded = mix(high ^ mix_int(int(seed) >> 32))
    folded = folded ^ torch.where(high != 0, mix(high ^ key), torch.zeros_like(high))
    hashed = mix((address & 0xFFFFFFFF) ^ folded ^ key)
    return ((hashed >> 8).float() + 0.5) / 16777216


def event_seed(seed, event):
    """64-bit read seed for a read event; random.py:26-27."""
    return (seed ^ mix_int(event & 0xFFFFFFFF)) | (mix_int(event >> 32) << 32)


def normal(address, seed, stream):
    """Box-Muller standard normal from streams (stream, stream+1); random.py:30-33."""
    first = uniform(address, seed, stream)
    second = uniform(address, seed, stream + 1)
    return torch.sqrt(-2 * torch.log(first)) * torch.cos((2 * math.pi) * second)


# ---------------------------------------------------------------------------
# Quantization and packing (memfast/quantization.py)
# ---------------------------------------------------------------------------
def grouped_quantize(value, bits, granularity, bw_e=None, *, signed=True):
    """Rectangular-group INT/BFP quantization; quantization.py:9-44."""
    dtype = torch.float64 if bits > 8 or bw_e is not None else torch.float32
    value = value.to(dtype)
    if not torch.isfinite(value).all():
        raise ValueError(f"quantized values must be finite in {dtype}")
    if not signed and ((value < 0).any() or bw_e is not None):
        raise ValueError("unsigned floating weights must be nonnegative INT values")
    rows, cols = value.shape
    gr = rows if granularity[0] is None else min(granularity[0], rows)
    gc = cols if granularity[1] is None else min(granularity[1], cols)
    nr, nc = math.ceil(rows / gr), math.ceil(cols / gc)
    blocks = F.pad(value, (0, nc * gc - cols, 0, nr * gr - rows)).reshape(nr, gr, nc, gc)
    peak = blocks.abs().amax((1, 3), keepdim=True)
    upper = (1 << (bits - int(signed))) - 1
    if bw_e is None:
        scale = torch.where(peak > 0, peak, 1.0) / upper
        tiny = torch.nextafter(torch.zeros((), dtype=dtype), torch.ones((), dtype=dtype))
        scale = scale.clamp_min(tiny)
        lower = -upper if signed else 0
    else:
        limit = (1 << (bw_e - 1)) - 1
        exponent = peak.clamp_min(torch.finfo(dtype).tiny).log2().floor()
        exponent = exponent.clamp(1 - limit, limit)
        scale = torch.pow(2.0, exponent + 2 - bits)
        lower = -(1 << (bits - 1))
    code = (blocks / scale).round().clamp_(lower, upper)
    code = code.reshape(nr * gr, nc * gc)[:rows, :cols].to(torch.int64)
    full = scale.expand(nr, gr, nc, gc).reshape(nr * gr, nc * gc)[:rows, :cols]
    return code, full


def read_starts(partitions, cfg):
    """Physical row index of every ADC read; quantization.py:76-79."""
    base = torch.arange(partitions)[:, None] * cfg.array_size[0]
    offsets = torch.arange(reads_per_array(cfg))[None] * read_rows(cfg)
    return (base + offsets).flatten()


def pack_weight(code, scale, cfg):
    """[K,O] codes -> packed [m,p,R,C] and per-read scales [m*Gr,p,C]; quantization.py:94-112."""
    k, o = code.shape
    r, c = cfg.array_size
    m, p = math.ceil(k / r), math.ceil(o / c)
    scale = scale.to(torch.float64 if is_wide(cfg) else torch.float32)
    padded = F.pad(code, (0, p * c - o, 0, m * r - k))
    store = torch.int64 if max(cfg.activation_bits, cfg.weight_bits) > 8 else torch.uint8
    packed = (padded & ((1 << cfg.weight_bits) - 1)).to(store)
    packed = packed.reshape(m, r, p, c).permute(0, 2, 1, 3).contiguous()
    grown = F.pad(scale[None, None], (0, p * c - o, 0, m * r - k), mode="replicate")[0, 0]
    scales = grown[read_starts(m, cfg)].reshape(m * reads_per_array(cfg), p, c).contiguous()
    return packed, scales


def weight_tiles(weight, cfg):
    """PyTorch-layout [O,K] weights -> packed tiles; quantization.py:82-91."""
    code, scale = grouped_quantize(
        weight.T.contiguous(), cfg.weight_bits, cfg.weight_quant_gran, cfg.bw_e,
        signed=cfg.weight_signed,
    )
    return pack_weight(code, scale, cfg)


def input_tiles(value, cfg, fixed_scale=None):
    """[N,K] inputs -> codes [N,m,R] and per-read scales [N,m*Gr]; quantization.py:115-137."""
    n, k = value.shape
    r = cfg.array_size[0]
    m = math.ceil(k / r)
    if fixed_scale is None:
        code, scale = grouped_quantize(value, cfg.activation_bits, cfg.input_quant_gran, cfg.bw_e)
    else:
        dtype = torch.float64 if is_wide(cfg) else torch.float32
        if not torch.isfinite(value).all():
            raise ValueError("quantized values must be finite")
        scale = fixed_scale.expand_as(value)
        upper = (1 << (cfg.activation_bits - 1)) - 1
        lower = -(1 << (cfg.activation_bits - 1)) if cfg.bw_e is not None else -upper
        code = (value.to(dtype) / scale).round().clamp(lower, upper).to(torch.int64)
    scale = scale.to(torch.float64 if is_wide(cfg) else torch.float32)
    padded = F.pad(code, (0, m * r - k))
    store = torch.int64 if max(cfg.activation_bits, cfg.weight_bits) > 8 else torch.uint8
    packed = (padded & ((1 << cfg.activation_bits) - 1)).to(store)
    scales = F.pad(scale[None], (0, m * r - k), mode="replicate")[0]
    scales = scales[:, read_starts(m, cfg)]
    return packed.reshape(n, m, r).contiguous(), scales.contiguous()


# ---------------------------------------------------------------------------
# Array model (memfast/reference.py)
# ---------------------------------------------------------------------------
def cell_addresses(m, p, w, r, c, begin, end):
    """Physical cell address (((i*p+t)*W+w)*R+r)*C+c; reference.py:14-19."""
    i = torch.arange(m)[:, None, None, None, None]
    t = torch.arange(begin, end)[None, :, None, None, None]
    b = torch.arange(w)[None, None, :, None, None]
    row = torch.arange(r)[None, None, None, :, None]
    col = torch.arange(c)[None, None, None, None, :]
    return (((i * p + t) * w + b) * r + row) * c + col


def restored(packed, cfg, seed, event, begin, end):
    """Programmed + read conductances [m,width,W,R,C]; reference.py:10-51."""
    ni = cfg.nonidealities
    m, p, r, c = packed.shape
    wl = weight_layout(cfg)
    w = len(wl)
    address = cell_addresses(m, p, w, r, c, begin, end)
    shifts = torch.tensor([e[0] for e in wl])[None, None, :, None, None]
    masks = torch.tensor([e[1] for e in wl])[None, None, :, None, None]
    state = (packed[:, begin:end, None].long() >> shifts) & masks
    dtype = torch.float64 if precise_currents(cfg) else torch.float32
    high, low = cfg.high_conductance, cfg.low_conductance
    raw = low + (high - low) * (state.to(dtype) / masks)
    binary = torch.where(
        state.bool(), torch.tensor(high, dtype=dtype), torch.tensor(low, dtype=dtype)
    )
    raw = torch.where(masks == 1, binary, raw).to(dtype)
    if ni.write_variation:
        raw = raw * torch.exp(ni.write_variation * normal(address, seed, 10))
    raw = raw * drift_factor(cfg)
    if ni.stuck_at_low + ni.stuck_at_high:
        sample = uniform(address, seed, 30)
        raw = torch.where(sample < ni.stuck_at_low, low, raw)
        band = (sample >= ni.stuck_at_low) & (sample < ni.stuck_at_low + ni.stuck_at_high)
        raw = torch.where(band, high, raw)
    read_seed = event_seed(seed, event)
    if ni.read_mode == "shared" and ni.read_variation:
        raw = raw * torch.exp(ni.read_variation * normal(address, read_seed, 20))
    return raw, address, read_seed


def adc(current, cfg, weight_slice=0):
    """Current -> ADC count (float, integer valued); reference.py:54-60."""
    ni = cfg.nonidealities
    peak = adc_maxima(cfg)[weight_slice]
    value = current * (1 / current_unit(cfg))
    if ni.adc_nonlinearity:
        value = value / (1 + ((ni.adc_nonlinearity / peak) * value).abs())
    return value.clamp(0, peak).round()


def partial(q, packed, cfg, seed, event, begin, end, *, conductance=None, codes=None):
    """Integer slice totals T [N, m*Gr, width, C]; reference.py:63-117.

    ``conductance`` injects the restored [m,width,W,R,C] tensor instead of
    sampling it (used for GPU parity under noise).  If ``codes`` is a dict it
    receives the per-(a,w) ADC counts as int64 [N, m*Gr, width, C] tensors.
    """
    ni = cfg.nonidealities
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    il, wl = input_layout(cfg), weight_layout(cfg)
    a_count, w_count = len(il), len(wl)
    width = end - begin
    raw, cell, read_seed = restored(packed, cfg, seed, event, begin, end)
    if conductance is not None:
        raw = conductance.to(raw.dtype)
    groups = reads_per_array(cfg)
    rows = read_rows(cfg)
    totals = torch.zeros((n, m, groups, width, c), dtype=torch.int64)
    vector = torch.arange(n)[:, None, None, None]
    array = torch.arange(m)[None, :, None, None]
    tile = torch.arange(begin, end)[None, None, :, None]
    col = torch.arange(c)[None, None, None, :]
    for ai, (ashift, amask, sa) in enumerate(il):
        voltage = ((q.long() >> ashift) & amask).to(raw.dtype) / amask * cfg.read_voltage
        if ni.voltage_variation:
            row = torch.arange(r)[None, None, :]
            address = ((vector[..., 0] * m + array[..., 0]) * a_count + ai) * r + row
            voltage *= 1 + ni.voltage_variation * normal(address, read_seed, 40)
        v = voltage.permute(1, 0, 2).contiguous()
        for wi, (_, wmask, sw) in enumerate(wl):
            g = raw[:, :, wi]
            if ni.read_mode == "slice_pair" and ni.read_variation:
                g = g * torch.exp(
                    ni.read_variation * normal(cell[:, :, wi] * a_count + ai, read_seed, 20)
                )
            for group in range(groups):
                start = group * rows
                stop = min(start + rows, r)
                length = stop - start
                sub_g, sub_v = g[:, :, start:stop], v[:, :, start:stop]
                effective = (sub_g - cfg.low_conductance).permute(0, 2, 1, 3)
                effective = effective.reshape(m, length, width * c)
                current = torch.bmm(sub_v, effective).permute(1, 0, 2).reshape(n, m, width, c)
                read_part = array * groups + group
                address = (
                    (((vector * m * groups + read_part) * p + tile) * a_count + ai) * w_count + wi
                ) * c + col
                if ni.read_mode == "output" and ni.read_variation:
                    base = sub_g.permute(0, 2, 1, 3).reshape(m, length, width * c)
                    sigma = ni.read_variation
                    mean = torch.bmm(sub_v, base) * math.expm1(0.5 * sigma**2)
                    variance = torch.bmm(sub_v.square(), base.square())
                    variance *= math.exp(sigma**2) * math.expm1(sigma**2)
                    mean = mean.permute(1, 0, 2).reshape_as(current)
                    variance = variance.permute(1, 0, 2).reshape_as(current)
                    current += mean + variance.sqrt() * normal(address, read_seed, 60)
                count = adc(current * (amask * wmask), cfg, wi).long()
                if codes is not None:
                    codes.setdefault((ai, wi), torch.zeros((n, m, groups, width, c), dtype=torch.int64))
                    codes[(ai, wi)][:, :, group] = count
                totals[:, :, group] += count * (sa * sw)
    dtype = torch.float64 if is_wide(cfg) else torch.float32
    return totals.reshape(n, m * groups, width, c).to(dtype)


def restore_scales(value, input_scale, weight_scale):
    """Overflow-safe FP64 value*xs*ws via frexp/ldexp; simulator.py:57-66."""
    vm, ve = torch.frexp(value.double())
    xm, xe = torch.frexp(input_scale.double())
    wm, we = torch.frexp(weight_scale.double())
    mantissa = vm * xm * wm
    exponent = ve + xe + we
    first = exponent.clamp(-1022, 1023)
    result = torch.ldexp(torch.ldexp(mantissa, first), exponent - first)
    return torch.where(mantissa == 0, 0.0, result)


def imported_tiles(codes, scales, cfg, zero_points=None):
    """``map_quantized`` programming of integer [O,K] weights (simulator.py:173-185, :399-425):
    packed codes, per-read scales and, with zero points, the per-read correction rows
    ``-(zero_point * scale)`` at each read's first row [m*Gr, O]."""
    o, k = codes.shape
    dtype = torch.float64 if is_wide(cfg) else torch.float32
    code = codes.to(torch.int64).T.contiguous()
    scale_full = scales.to(dtype).expand(o, k).T.contiguous()
    packed, wscale = pack_weight(code, scale_full, cfg)
    if zero_points is None:
        return packed, wscale, None
    zeros = zero_points.to(dtype).expand(o, k).T.contiguous()
    starts = read_starts(math.ceil(k / cfg.array_size[0]), cfg).clamp_max(k - 1)
    return packed, wscale, -(zeros[starts] * scale_full[starts])


def zero_point_correction(output, q, xscale, correction, cfg, stable=False):
    """Add the digital zero-point term of simulator.py:587-611 to ``output`` [N, O]: each
    read's signed input code sum times its input scale times the correction row, in FP32
    as one matrix product, or per chunk of C columns with restore_scales in FP64."""
    bits = cfg.activation_bits
    signed = q.to(torch.int64).reshape(q.shape[0], -1) & ((1 << bits) - 1)
    signed = (signed ^ (1 << (bits - 1))) - (1 << (bits - 1))
    rows, step = cfg.array_size[0], read_rows(cfg)
    padded = F.pad(signed.reshape(q.shape[0], -1, rows), (0, reads_per_array(cfg) * step - rows))
    sums = padded.reshape(q.shape[0], -1, step).sum(-1)
    if is_wide(cfg) or stable:
        output = output.clone()
        c = cfg.array_size[1]
        for begin in range(0, output.shape[1], c):
            end = min(begin + c, output.shape[1])
            output[:, begin:end] += restore_scales(sums[:, :, None], xscale[:, :, None],
                                                   correction[None, :, begin:end]).sum(1)
        return output
    dtype = output.dtype
    return output + (sums.to(dtype) * xscale.to(dtype)) @ correction.to(dtype)


def execute(q, xscale, packed, wscale, cfg, seed, event, out_features, *, bias=None,
            arrays=2, stable=False, conductance=None, totals=None, tiles=None,
            zero_correction=None):
    """Fused epilogue of AnalogMatrix._execute (simulator.py:561-616).

    ``conductance`` (optional) is the full [m,p,W,R,C] injected tensor.
    ``totals`` (optional) supplies the slice totals [N, m*Gr, p, C] of every
    tile instead of computing them with ``partial`` (to check a kernel's
    epilogue on its own totals).  ``tiles`` = (begin, end), with ``begin`` a
    multiple of ``arrays``, runs only the chunks of those tiles (same per-chunk
    arithmetic, since each output column depends only on its own chunk) and
    returns their [N, (end-begin)*C] columns, before bias and the FP64 retry.
    Zero-point correction (map_quantized) is not covered by the hot path.
    """
    p = packed.shape[1]
    c = cfg.array_size[1]
    wide = is_wide(cfg) or stable
    output = torch.empty((q.shape[0], p * c), dtype=torch.float64 if wide else torch.float32)
    width = min(arrays, p)
    first, last = (0, p) if tiles is None else tiles
    if first % width or not 0 <= first < last <= p:
        raise ValueError("tiles must start on a chunk boundary and lie within [0, p]")
    for begin in range(first, last, width):
        end = min(begin + width, p)
        injected = None if conductance is None else conductance[:, begin:end]
        if totals is not None:
            value = totals[:, :, begin:end].to(torch.float64 if is_wide(cfg) else torch.float32)
        else:
            value = partial(q, packed, cfg, seed, event, begin, end, conductance=injected)
        if wide:
            value = restore_scales(value, xscale[:, :, None, None], wscale[None, :, begin:end, :])
        else:
            value = value * xscale[:, :, None, None]
            value = value * wscale[None, :, begin:end, :]
        output[:, begin * c:end * c] = value.sum(1).flatten(1)
    if tiles is not None:
        return output[:, first * c:min(last, end) * c].contiguous()
    output = output[:, :out_features].contiguous()
    if zero_correction is not None:
        output = zero_point_correction(output, q, xscale, zero_correction, cfg, stable)
    if bias is not None:
        output = output + bias
    if not is_wide(cfg) and not stable and not torch.isfinite(output).all():
        return execute(q, xscale, packed, wscale, cfg, seed, event, out_features, bias=bias,
                       arrays=arrays, stable=True, conductance=conductance, totals=totals,
                       zero_correction=zero_correction)
    return output


def mm(a, b, cfg, *, name="matrix.0", event=0, conductance=None):
    """``Simulator(cfg, device='cpu').mm(a, b)`` on a fresh simulator.

    Follows functional.mm -> Simulator._matrix_for -> AnalogMatrix.__init__ ->
    AnalogMatrix.forward (functional.py:130-208, simulator.py:133-171,
    :353-430, :618-646): B is programmed as ``matrix.{k}``, A is quantized
    per call, the output is cast back to A's dtype.
    """
    a = a.detach().cpu()
    b = b.detach().cpu()
    k, o = b.shape
    packed, wscale = weight_tiles(b.T, cfg)
    seed = name_seed(cfg.seed, name)
    q, xscale = input_tiles(a.reshape(-1, k), cfg)
    out = execute(q, xscale, packed, wscale, cfg, seed, event, o, conductance=conductance)
    return out.reshape(*a.shape[:-1], o).to(a.dtype)


def ideal_totals_closed_form(q, packed, cfg, begin=0, end=None):
    """T for ideal devices from integer digits: sum_aw fa*fw*min(sum_r da*dw, max_w).

    An independent restatement of the ideal ADC (docs/user-guide.md:330-345)
    used to pin ``partial`` when every nonideality is off.
    """
    n, m, r = q.shape
    p, c = packed.shape[1], cfg.array_size[1]
    end = p if end is None else end
    groups, rows = reads_per_array(cfg), read_rows(cfg)
    maxima = adc_maxima(cfg)
    totals = torch.zeros((n, m, groups, end - begin, c), dtype=torch.int64)
    for (sa_, ma, fa) in input_layout(cfg):
        da = (q.long() >> sa_) & ma  # [n, m, r]
        for wi, (sw_, mw, fw) in enumerate(weight_layout(cfg)):
            dw = (packed[:, begin:end].long() >> sw_) & mw  # [m, t, r, c]
            for j in range(groups):
                lo, hi = j * rows, min((j + 1) * rows, r)
                s = torch.einsum("nir,itrc->nitc", da[:, :, lo:hi], dw[:, :, lo:hi])
                totals[:, :, j] += fa * fw * s.clamp_max(maxima[wi])
    return totals.reshape(n, m * groups, end - begin, c)
