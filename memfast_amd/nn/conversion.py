"""``convert_model``: replace a model's layers by analog layers (memfast/nn/conversion.py).

Selection (``_Selection``):
* ``include=None`` selects everything, an empty sequence nothing; a path selects its
  whole subtree and ``""`` the root; ``exclude`` wins and covers descendants too;
  unknown paths, and paths inside an already converted layer, raise;
* a module reachable under several names converts only if every one of its names is
  included and none excluded; it is replaced once, so sharing is preserved.

Conversion (``_Converter``) walks the (copied, unless ``inplace``) model depth first and
builds each selected layer with the builder of its type (``_BUILDERS``).  Existing analog
layers are kept as they are, after checks that they match the simulator's
configuration, mode and device.  ``training=True`` builds trainable layers that share
the model's own Parameters (ties between layers survive).  Llama subtrees that gain
analog Linear layers get ``pretraining_tp=1``: the tensor-partition path reads
``.weight`` directly and would bypass the analog projections.  The default result is in
eval mode without gradients.
"""

import copy

from torch import nn

from ..simulator import AnalogMatrix
from .convolution import AnalogConv2d
from .linear import AnalogLinear
from .recurrent import AnalogGRU, AnalogGRUCell, AnalogRNN, AnalogRNNCell
from .training import TrainableAnalogConv2d, TrainableAnalogLinear, _validate_gradient_mode

_RECURRENT = (AnalogRNN, AnalogRNNCell, AnalogGRU, AnalogGRUCell)
_ANALOG = (AnalogMatrix, AnalogConv2d) + _RECURRENT
_TRAINABLE = (TrainableAnalogLinear, TrainableAnalogConv2d)
_CONVERTED = _ANALOG + _TRAINABLE


# ---------------------------------------------------------------------------
# Builders of analog layers, by the digital layer's type
# ---------------------------------------------------------------------------
def _linear(module, simulator, name, training, gradient_mode):
    if training:
        return TrainableAnalogLinear(module, simulator, name=name or "linear",
                                     gradient_mode=gradient_mode)
    return AnalogLinear(module, simulator, name=name or "linear")


def _conv(module, simulator, name, training, gradient_mode):
    if training:
        return TrainableAnalogConv2d(module, simulator, name=name or "conv",
                                     gradient_mode=gradient_mode)
    return AnalogConv2d(module, simulator, name=name or "conv")


def _recurrent(analog_type, default_name):
    def build(module, simulator, name, training, gradient_mode):
        return analog_type(module, simulator, training=training, name=name or default_name,
                           gradient_mode=gradient_mode)
    return build


_BUILDERS = (
    (nn.Linear, _linear),
    (nn.Conv2d, _conv),
    (nn.RNNCell, _recurrent(AnalogRNNCell, "rnn_cell")),
    (nn.GRUCell, _recurrent(AnalogGRUCell, "gru_cell")),
    (nn.RNN, _recurrent(AnalogRNN, "rnn")),
    (nn.GRU, _recurrent(AnalogGRU, "gru")),
)
_SUPPORTED = tuple(kind for kind, _ in _BUILDERS)


def _builder(module):
    return next((build for kind, build in _BUILDERS if isinstance(module, kind)), None)


# ---------------------------------------------------------------------------
# Shared Parameters of trainable conversions
# ---------------------------------------------------------------------------
def _share_cell(cell, source, suffix=""):
    """Point a trainable cell's projections at ``source``'s Parameters (PyTorch names
    ``weight_ih{suffix}`` and so on) and expose them under the cell's own names."""
    for projection, kind in ((cell.input, "ih"), (cell.hidden, "hh")):
        projection.weight = getattr(source, f"weight_{kind}{suffix}")
        projection.bias = getattr(source, f"bias_{kind}{suffix}", None)
        cell.register_parameter(f"weight_{kind}", projection.weight)
        cell.register_parameter(f"bias_{kind}", projection.bias)


def _share_parameters(result, source):
    if isinstance(result, _TRAINABLE):
        result.weight, result.bias = source.weight, source.bias
    elif isinstance(result, (AnalogRNNCell, AnalogGRUCell)):
        _share_cell(result, source)
    elif isinstance(result, (AnalogRNN, AnalogGRU)):
        directions = 2 if result.bidirectional else 1
        for index, cell in enumerate(result.cells):
            layer, reverse = divmod(index, directions)
            suffix = f"_l{layer}" + ("_reverse" if reverse else "")
            _share_cell(cell, source, suffix)
            for parameter in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                result.register_parameter(parameter + suffix, getattr(cell, parameter))


def _disable_tensor_partitions(module):
    """``pretraining_tp=1`` for a Llama module whose subtree holds analog Linear layers."""
    config = getattr(module, "config", None)
    if (getattr(config, "model_type", None) == "llama" and getattr(config, "pretraining_tp", 1) > 1
            and any(isinstance(m, (AnalogLinear, TrainableAnalogLinear)) for m in module.modules())):
        config.pretraining_tp = 1


# ---------------------------------------------------------------------------
# Selection
# ---------------------------------------------------------------------------
def _path_set(value, label):
    if isinstance(value, str):
        raise TypeError(f"{label} must be a sequence of module paths")
    try:
        paths = tuple(value)
    except TypeError:
        raise TypeError(f"{label} must be a sequence of module paths") from None
    if not all(isinstance(path, str) for path in paths):
        raise TypeError(f"{label} module paths must be strings")
    return set(paths)


def _under(paths, name):
    """Whether module path ``name`` lies in the subtree of any of ``paths``."""
    return any(path == "" or name == path or name.startswith(path + ".") for path in paths)


class _Selection:
    """The include/exclude paths of a conversion, checked against the model."""

    def __init__(self, model, include, exclude):
        self.included = None if include is None else _path_set(include, "include")
        self.excluded = _path_set(exclude, "exclude")
        modules = dict(model.named_modules(remove_duplicate=False))
        for label, paths in (("included", self.included), ("excluded", self.excluded)):
            paths = paths or set()
            unknown = paths - modules.keys()
            if unknown:
                raise ValueError(f"unknown {label} modules: {sorted(unknown)}")
            for path in paths:
                self._reject_inside_converted(modules, path)

    @staticmethod
    def _reject_inside_converted(modules, path):
        parts = path.split(".")
        ancestors = (".".join(parts[:depth]) for depth in range(len(parts)))
        for ancestor in ancestors:
            if ancestor != path and isinstance(modules[ancestor], _CONVERTED):
                raise ValueError(f"{path}: selection inside a converted layer is unsupported; "
                                 f"select its path {ancestor!r}")

    def resolve(self, target):
        """(ids of excluded modules, ids of selected modules) of ``target``: a module is
        selected when all of its names are included and none is excluded."""
        names = {}
        for name, module in target.named_modules(remove_duplicate=False):
            names.setdefault(id(module), []).append(name)
        excluded = {key for key, aliases in names.items()
                    if any(_under(self.excluded, name) for name in aliases)}
        selected = {key for key, aliases in names.items() if key not in excluded
                    and (self.included is None
                         or all(_under(self.included, name) for name in aliases))}
        return excluded, selected


def _check_target(target, simulator, selected, training):
    """Reject what cannot convert, before anything is built."""
    inside = {id(child) for layer in target.modules() if isinstance(layer, _CONVERTED)
              for child in layer.modules() if child is not layer}
    for name, module in target.named_modules():
        if isinstance(module, AnalogMatrix) and module.simulator.device != simulator.device:
            raise ValueError(f"{name}: existing analog matrices are bound to their simulator device")
        if id(module) in inside or id(module) not in selected:
            continue
        if isinstance(module, nn.Conv2d) and isinstance(module.padding, str):
            raise ValueError(f"{name}: numeric Conv2d padding is required")
        if not isinstance(module, _CONVERTED):
            continue
        if (training and isinstance(module, _ANALOG)
                and not getattr(module, "_hardware_aware_training", False)):
            raise ValueError("training conversion requires the original digital layer weights")
        mismatched = any(isinstance(child, AnalogMatrix)
                         and (child.config != simulator.config
                              or child.simulator.mode != simulator.mode)
                         for child in module.modules())
        if mismatched:
            raise ValueError(f"{name}: reconversion requires matching physical config and mode")


class _Converter:
    """Depth-first replacement of selected layers; each module is converted once."""

    def __init__(self, simulator, excluded, selected, training, gradient_mode):
        self.simulator, self.training, self.gradient_mode = simulator, training, gradient_mode
        self.excluded, self.selected = excluded, selected
        self.done = {}

    def __call__(self, module, name):
        key = id(module)
        if key in self.excluded or (isinstance(module, _SUPPORTED + _CONVERTED)
                                    and key not in self.selected):
            return module
        if isinstance(module, _CONVERTED):
            return self._keep_converted(module)
        if key in self.done:
            return self.done[key]
        build = _builder(module)
        if build is None:
            self.done[key] = module
            self._convert_children(module, name)
            _disable_tensor_partitions(module)
            return module
        result = build(module, self.simulator, name, self.training, self.gradient_mode)
        if self.training:
            _share_parameters(result, module)
        self.done[key] = result
        return result

    def _convert_children(self, module, name):
        for attribute, child in list(module._modules.items()):
            if child is not None:
                setattr(module, attribute, self(child, f"{name}.{attribute}" if name else attribute))

    def _keep_converted(self, module):
        """An existing analog layer stays; under ``training`` its trainable parts take the
        requested gradient mode."""
        if not self.training:
            return module
        if isinstance(module, _ANALOG) and not getattr(module, "_hardware_aware_training", False):
            raise ValueError("training conversion requires the original digital layer weights")
        for part in module.modules():
            if isinstance(part, _TRAINABLE + _RECURRENT):
                part.gradient_mode = self.gradient_mode
        return module


def convert_model(model, simulator, *, include=None, exclude=(), inplace=False, training=False,
                  gradient_mode="quantized"):
    """Convert Linear, Conv2d, RNN/GRU cells and sequences to analog execution."""
    if not isinstance(model, nn.Module):
        raise TypeError("model must be a PyTorch module")
    if not isinstance(training, bool):
        raise TypeError("training must be a boolean")
    _validate_gradient_mode(gradient_mode)
    selection = _Selection(model, include, exclude)
    target = model if inplace else copy.deepcopy(model)
    excluded, selected = selection.resolve(target)
    _check_target(target, simulator, selected, training)
    target.to(simulator.device)
    converted = _Converter(simulator, excluded, selected, training, gradient_mode)(target, "")
    return converted.train() if training else converted.eval().requires_grad_(False)


def reset_read_events(model, event=0):
    """Set the read event of every programmed matrix, hardware-aware layers included."""
    for module in model.modules():
        if isinstance(module, AnalogMatrix):
            module.reset_read(event)
