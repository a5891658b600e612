"""Checkpoint state of a programmed matrix: validation on load and the extra state.

A programmed matrix (``AnalogMatrix``) saves its program as buffers, ``packed``,
``weight_scale``, optional ``zero_correction`` and ``input_scale``, and ``bias``, plus an
extra state of configuration, logical dimensions, sampling name, seed and read event.
Loading must reject anything that could not have been produced under the simulator's
own configuration, with the reference's messages (memfast/simulator.py:452-534):

* before torch copies the tensors: integer codes within ``weight_bits`` and finite,
  nonnegative scales;
* after the copy: finite scales and bias in the reconstruction dtype, a fixed input
  scale that still satisfies the read grouping, a well-shaped finite zero-point
  correction;
* extra state: matching logical dimensions, no removed noise model, the same physical
  configuration (fields that older checkpoints lack take their defaults), a 32-bit seed
  and a valid read event.
"""

import json
from dataclasses import asdict

import torch

_CODE_DTYPES = (torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64)
_OPTIONAL_BUFFERS = ("input_scale", "zero_correction")
# Config fields added after the first checkpoints were written, with their defaults.
_LATER_FIELDS = dict(rows_per_read=None, input_slice=None, weight_slice=None, bw_e=None,
                     weight_signed=True)


def _finite_nonnegative(tensor):
    return bool(torch.isfinite(tensor).all()) and not bool((tensor < 0).any())


def check_incoming(matrix, state_dict, prefix):
    """Checks on the serialized tensors, before they are copied into ``matrix``."""
    packed = state_dict.get(prefix + "packed")
    if packed is not None:
        if not torch.is_tensor(packed) or packed.dtype not in _CODE_DTYPES:
            raise ValueError("checkpoint packed weights must have an integer dtype")
        codes = packed.to(torch.int64)
        limit = 1 << matrix.config.weight_bits
        if codes.numel() and not (0 <= int(codes.min()) and int(codes.max()) < limit):
            raise ValueError("checkpoint packed weights exceed the configured bit width")
    scales = state_dict.get(prefix + "weight_scale")
    if scales is not None and not (torch.is_tensor(scales) and scales.is_floating_point()
                                   and _finite_nonnegative(scales)):
        raise ValueError("checkpoint weight scales must be finite and nonnegative")


def shape_optional_buffers(matrix, state_dict, prefix):
    """Give absent optional buffers the serialized shape, so torch can copy into them."""
    for name in _OPTIONAL_BUFFERS:
        key = prefix + name
        if key in state_dict and matrix._buffers[name] is None:
            matrix._buffers[name] = torch.empty_like(state_dict[key], device=matrix.packed.device)


def check_loaded(matrix):
    """Checks of the copied buffers in their reconstruction dtype."""
    if not _finite_nonnegative(matrix.weight_scale):
        raise ValueError("checkpoint weight scales exceed the reconstruction dtype")
    if matrix.bias is not None and not bool(torch.isfinite(matrix.bias).all()):
        raise ValueError("checkpoint bias exceeds the reconstruction dtype")
    if matrix.input_scale is not None:
        matrix.set_input_scale(matrix.input_scale)    # re-validates the read grouping
    correction = matrix.zero_correction
    if correction is not None:
        if tuple(correction.shape) != (matrix.weight_scale.shape[0], matrix.out_features):
            raise ValueError("checkpoint zero-point correction has an invalid shape")
        if not bool(torch.isfinite(correction).all()):
            raise ValueError("checkpoint zero-point correction must be finite")


def extra_state(matrix):
    """The extra state a programmed matrix saves (memfast/simulator.py:495-503)."""
    return dict(config=asdict(matrix.config), in_features=matrix.in_features,
                out_features=matrix.out_features, name=matrix.name, seed=matrix.seed,
                event=matrix._event)


def _normalized(config):
    """A serialized Config with tuples and lists made alike (JSON-loaded checkpoints)."""
    return json.loads(json.dumps(config))


def saved_config_matches(saved, config):
    """Whether a checkpoint's serialized Config describes ``config``.  A removed noise
    model raises; fields older checkpoints lack take their defaults."""
    effects = dict(saved["nonidealities"])
    if effects.pop("output_noise", 0) != 0:
        raise ValueError("checkpoint uses a removed noise model")
    restated = {**_LATER_FIELDS, **saved, "nonidealities": effects}
    return _normalized(restated) == _normalized(asdict(config))


def check_extra_state(matrix, state):
    """Validate a checkpoint's extra state against ``matrix``; returns (name, seed, event)."""
    for key in ("in_features", "out_features"):
        if key in state and (type(state[key]) is not int or state[key] != getattr(matrix, key)):
            raise ValueError("checkpoint logical matrix dimensions differ")
    if not saved_config_matches(state["config"], matrix.config):
        raise ValueError("checkpoint physical configuration differs")
    seed = state["seed"]
    if type(seed) is not int or not 0 <= seed < 1 << 32:
        raise ValueError("invalid checkpoint sampling seed")
    return state["name"], seed, state["event"]
