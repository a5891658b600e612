"""Validated array geometry, quantization, slicing and device nonidealities.

Drop-in for the reference's ``memfast/config.py``: the dataclass fields, their
defaults, the derived properties and the cases that raise ``ValueError`` follow
``Nonidealities`` (memfast/config.py:21-45) and ``Config`` (memfast/config.py:48-224).

Derived layouts are least-significant-slice first.  Each entry is
``(shift, mask, factor)``: the slice digit is ``(code >> shift) & mask`` and it
contributes ``factor * digit`` to the signed (two's complement) integer code.
The most significant slice of a signed code carries factor ``-(1 << shift)``.
"""

import math
import struct
from dataclasses import dataclass, fields
from functools import cached_property

_FP32_MAX = 3.4028234663852886e38
_FP32_MIN_SUBNORMAL = 1.401298464324817e-45


def _check_int(value, name, low, high):
    # bool is an int subclass; the reference accepts exact ints only.
    if type(value) is not int or value < low or value > high:
        raise ValueError(f"{name} must be an integer in [{low}, {high}]")


def _check_nonnegative(value, name):
    ok = isinstance(value, (int, float)) and not isinstance(value, bool)
    if not ok or not math.isfinite(value) or value < 0:
        raise ValueError(f"{name} must be a finite nonnegative number")


def _to_fp32(value):
    return struct.unpack("f", struct.pack("f", value))[0]


@dataclass(frozen=True)
class Nonidealities:
    """Noise magnitudes (dimensionless) and retention times (seconds).

    Mirrors memfast/config.py:21-45: every numeric field is finite and
    nonnegative, ``read_mode`` is one of shared/slice_pair/output, stuck-at
    probabilities sum to at most one and the drift reference time is positive.
    """

    write_variation: float = 0.02
    read_variation: float = 0.0
    read_mode: str = "shared"
    voltage_variation: float = 0.0
    adc_nonlinearity: float = 0.0
    stuck_at_low: float = 0.0
    stuck_at_high: float = 0.0
    drift_coefficient: float = 0.0
    drift_time: float = 0.0
    drift_reference_time: float = 1.0

    def __post_init__(self):
        for item in fields(self):
            if item.name == "read_mode":
                continue
            _check_nonnegative(getattr(self, item.name), item.name)
        if self.read_mode not in READ_MODES:
            raise ValueError("read_mode must be shared, slice_pair, or output")
        if self.stuck_at_low + self.stuck_at_high > 1:
            raise ValueError("stuck-at probabilities must sum to at most one")
        if self.drift_reference_time <= 0:
            raise ValueError("drift_reference_time must be positive")

    @property
    def drift_factor(self):
        """Power-law retention multiplier applied to every programmed cell."""
        return (1 + self.drift_time / self.drift_reference_time) ** (-self.drift_coefficient)

    @property
    def ideal(self):
        """True when every device effect is off, so ADC counts have a closed form."""
        return (
            self.write_variation == 0
            and self.read_variation == 0
            and self.voltage_variation == 0
            and self.adc_nonlinearity == 0
            and self.stuck_at_low == 0
            and self.stuck_at_high == 0
            and self.drift_factor == 1.0
        )


READ_MODES = ("shared", "slice_pair", "output")


def _slice_widths(value, name, bits, signed):
    """Normalise a slice-width sequence (MSB first) or raise ValueError."""
    try:
        items = tuple(value)
        if any(isinstance(item, bool) for item in items):
            raise ValueError
        widths = tuple(int(item.__index__()) for item in items)
    except (TypeError, ValueError, AttributeError):
        raise ValueError(f"{name} must contain integer slice widths") from None
    if not widths or sum(widths) != bits:
        raise ValueError(f"{name} slice widths must sum to {bits}")
    if signed and widths[0] != 1:
        raise ValueError(f"{name} must start with a one-bit sign slice and sum to {bits}")
    if min(widths) < 1 or max(widths) > 16:
        raise ValueError(f"{name} slice widths must be in [1,16]")
    return widths


def layout(widths, bits, signed=True):
    """LSB-first ``(shift, mask, factor)`` entries for MSB-first slice widths.

    ``None`` means one-bit slices.  Follows memfast/config.py:193-201.
    """
    widths = (1,) * bits if widths is None else tuple(widths)
    entries = []
    shift = 0
    count = len(widths)
    for position, width in enumerate(widths[::-1]):
        weight = 1 << shift
        if signed and position == count - 1:
            weight = -weight
        entries.append((shift, (1 << width) - 1, weight))
        shift += width
    return tuple(entries)


@dataclass(frozen=True)
class Config:
    """Physical matrices use [reduction rows K, output columns O] coordinates.

    Activations are signed two's complement codes.  ``weight_signed=False``
    selects unsigned INT weight codes whose slices all carry positive factors.
    Fields, defaults and validation follow memfast/config.py:48-165.
    """

    activation_bits: int = 8
    weight_bits: int = 8
    array_size: tuple = (64, 64)
    weight_quant_gran: tuple = (None, 1)
    input_quant_gran: tuple = (1, None)
    adc_bits: object = 6
    high_conductance: float = 1e-5
    low_conductance: float = 1e-7
    read_voltage: float = 0.2
    seed: int = 135
    nonidealities: Nonidealities = Nonidealities()
    rows_per_read: object = None
    input_slice: object = None
    weight_slice: object = None
    bw_e: object = None
    weight_signed: bool = True

    def __hash__(self):
        """The hash of the field values (what the generated ``__hash__`` computes), kept after
        the first call: the instance is frozen and the lookup caches keyed by it hash it on
        every read."""
        cached = self.__dict__.get("_hash")
        if cached is None:
            cached = hash(tuple(getattr(self, field.name) for field in fields(self)))
            object.__setattr__(self, "_hash", cached)
        return cached

    def __getstate__(self):
        # String hashes differ between processes: a pickled copy computes its own.
        state = dict(self.__dict__)
        state.pop("_hash", None)
        return state

    def __post_init__(self):
        _check_int(self.activation_bits, "activation_bits", 2, 32)
        _check_int(self.weight_bits, "weight_bits", 2, 32)
        if type(self.weight_signed) is not bool:
            raise ValueError("weight_signed must be a boolean")
        if self.bw_e is not None:
            _check_int(self.bw_e, "bw_e", 2, 11)
            if not self.weight_signed:
                raise ValueError("unsigned weights require INT quantization (bw_e=None)")
        if self.input_slice is not None:
            widths = _slice_widths(self.input_slice, "input_slice", self.activation_bits, True)
            object.__setattr__(self, "input_slice", widths)
        if self.weight_slice is not None:
            widths = _slice_widths(
                self.weight_slice, "weight_slice", self.weight_bits, self.weight_signed
            )
            object.__setattr__(self, "weight_slice", widths)
        if isinstance(self.adc_bits, (tuple, list)):
            widths = tuple(self.adc_bits)
            if len(widths) != len(self.weight_layout):
                raise ValueError("adc_bits must have one entry per weight slice, MSB first")
            for width in widths:
                _check_int(width, "adc_bits", 1, 16)
            object.__setattr__(self, "adc_bits", widths)
        else:
            _check_int(self.adc_bits, "adc_bits", 1, 16)
        if self.reconstruction_bound > 2**63 - 1:
            raise ValueError(
                "slice reconstruction exceeds the signed 64-bit accumulator; "
                "reduce precision, ADC bits, or use wider multibit slices"
            )
        _check_int(self.seed, "seed", 0, 2**32 - 1)
        for name in ("array_size", "weight_quant_gran", "input_quant_gran"):
            pair = getattr(self, name)
            if not isinstance(pair, tuple) or len(pair) != 2:
                raise ValueError(f"{name} must be a pair")
            for value in pair:
                if value is None and name != "array_size":
                    continue
                _check_int(value, name, 1, 65536)
        rows, columns = self.array_size
        if self.rows_per_read is not None:
            _check_int(self.rows_per_read, "rows_per_read", 1, rows)
        if columns % 4:
            raise ValueError("array columns must be divisible by four")
        for group in (self.weight_quant_gran[0], self.input_quant_gran[1]):
            if group is None or group % rows == 0:
                continue
            if rows % self.read_rows or group % self.read_rows:
                raise ValueError(
                    "reduction scale groups must align with every ADC read boundary; "
                    "use a multiple of array rows, or a multiple of rows_per_read "
                    "when it divides array rows"
                )
        for name in ("high_conductance", "low_conductance", "read_voltage"):
            value = getattr(self, name)
            _check_nonnegative(value, name)
            if value <= 0:
                raise ValueError(f"{name} must be positive")
        if self.high_conductance <= self.low_conductance:
            raise ValueError("high_conductance must exceed low_conductance")
        try:
            high = _to_fp32(self.high_conductance)
            low = _to_fp32(self.low_conductance)
        except OverflowError:
            raise ValueError("conductances must be representable in FP32") from None
        if not 0 < low < high <= _FP32_MAX:
            raise ValueError("conductances must remain distinct and positive in FP32")
        if not _FP32_MIN_SUBNORMAL <= self.read_voltage <= _FP32_MAX:
            raise ValueError("read_voltage must be representable in FP32")
        if not 1 / _FP32_MAX <= self.current_unit <= _FP32_MAX:
            raise ValueError("current unit and reciprocal must be representable in FP32")
        if not isinstance(self.nonidealities, Nonidealities):
            raise TypeError("nonidealities must be Nonidealities")

    # -- derived geometry (memfast/config.py:167-224) -------------------------
    # Layouts and flags are computed once per (immutable) Config.
    @property
    def current_unit(self):
        """Current of one ideal digit product: (H - L) * V_read."""
        return (self.high_conductance - self.low_conductance) * self.read_voltage

    @cached_property
    def adc_maxima(self):
        """Largest ADC count per weight slice, LSB-first (adc_bits is MSB-first)."""
        count = len(self.weight_layout)
        if type(self.adc_bits) is int:
            widths = (self.adc_bits,) * count
        else:
            widths = tuple(self.adc_bits)[::-1]
        return tuple((1 << width) - 1 for width in widths)

    @property
    def adc_maximum(self):
        return max(self.adc_maxima)

    @property
    def read_rows(self):
        """Rows summed before each ADC conversion (P)."""
        return self.array_size[0] if self.rows_per_read is None else self.rows_per_read

    @property
    def reads_per_array(self):
        """ADC reads per physical array (Gr = ceil(R / P))."""
        return -(-self.array_size[0] // self.read_rows)

    @staticmethod
    def _layout(widths, bits, signed=True):
        return layout(widths, bits, signed)

    @cached_property
    def input_layout(self):
        return layout(self.input_slice, self.activation_bits, True)

    @cached_property
    def weight_layout(self):
        return layout(self.weight_slice, self.weight_bits, self.weight_signed)

    @property
    def reconstruction_bound(self):
        """Largest |slice total| the signed shift-add can reach."""
        inputs = sum(abs(entry[2]) for entry in self.input_layout)
        weights = sum(
            abs(entry[2]) * maximum for entry, maximum in zip(self.weight_layout, self.adc_maxima)
        )
        return inputs * weights

    @cached_property
    def wide(self):
        """FP64 scale restoration and 64-bit codes (precision > 8 or BFP)."""
        return max(self.activation_bits, self.weight_bits) > 8 or self.bw_e is not None

    @property
    def wide_codes(self):
        return max(self.activation_bits, self.weight_bits) > 8

    @cached_property
    def precise_currents(self):
        """FP64 currents where FP32 rounding could move ideal ADC counts."""
        widest = max(entry[1] for entry in (*self.input_layout, *self.weight_layout))
        high, low, volt = self.high_conductance, self.low_conductance, self.read_voltage
        return (
            widest > 255
            or high - low < high * 1e-4
            or high * volt * self.read_rows > 8e37
            or min(low, volt) < 1e-18
            or max(high, volt) > 1e18
        )


__all__ = ["Config", "Nonidealities", "layout", "READ_MODES"]
