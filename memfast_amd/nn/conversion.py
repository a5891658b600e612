"""Model conversion with explicit selection and shared-module semantics.

Restates memfast/nn/conversion.py:
* ``include=None`` selects everything, an empty sequence nothing; a path
  selects its whole subtree and ``""`` the root; ``exclude`` wins and also
  covers descendants; unknown paths raise;
* a module reachable under several names converts only if every alias is
  included and none excluded, and is replaced once (identity preserved);
* existing analog layers are atomic and must match the simulator's config,
  mode and device; ``training=True`` keeps trainable master parameters;
* Llama subtrees with analog Linear layers get ``pretraining_tp=1`` so their
  projections are actually invoked.
The default returns a converted deep copy in eval mode without gradients.
"""

import copy

from torch import nn

from ..simulator import AnalogMatrix
from .convolution import AnalogConv2d
from .linear import AnalogLinear
from .recurrent import AnalogGRU, AnalogGRUCell, AnalogRNN, AnalogRNNCell
from .training import TrainableAnalogConv2d, TrainableAnalogLinear, _validate_gradient_mode

_ANALOG = (AnalogMatrix, AnalogConv2d, AnalogRNN, AnalogRNNCell, AnalogGRU, AnalogGRUCell)
_TRAINABLE = (TrainableAnalogLinear, TrainableAnalogConv2d)
_SUPPORTED = (nn.Linear, nn.Conv2d, nn.RNNCell, nn.RNN, nn.GRUCell, nn.GRU)


def _paths(value, name):
    if isinstance(value, str):
        raise TypeError(f"{name} must be a sequence of module paths")
    try:
        items = tuple(value)
    except TypeError:
        raise TypeError(f"{name} must be a sequence of module paths") from None
    if any(not isinstance(item, str) for item in items):
        raise TypeError(f"{name} module paths must be strings")
    return set(items)


def _covers(paths, name):
    return any(path == "" or name == path or name.startswith(path + ".") for path in paths)


def convert_model(model, simulator, *, include=None, exclude=(), inplace=False, training=False,
                  gradient_mode="quantized"):
    """Convert Linear, Conv2d, RNN/GRU cells and sequences to analog execution."""
    if not isinstance(model, nn.Module):
        raise TypeError("model must be a PyTorch module")
    if not isinstance(training, bool):
        raise TypeError("training must be a boolean")
    _validate_gradient_mode(gradient_mode)
    included = None if include is None else _paths(include, "include")
    excluded = _paths(exclude, "exclude")
    by_path = dict(model.named_modules(remove_duplicate=False))
    for label, selection in (("included", included), ("excluded", excluded)):
        missing = (selection or set()) - by_path.keys()
        if missing:
            raise ValueError(f"unknown {label} modules: {sorted(missing)}")
        for path in selection or ():
            parts = path.split(".")
            for depth in range(len(parts)):
                ancestor = ".".join(parts[:depth])
                if ancestor != path and isinstance(by_path[ancestor], _ANALOG + _TRAINABLE):
                    raise ValueError(
                        f"{path}: selection inside a converted layer is unsupported; "
                        f"select its path {ancestor!r}"
                    )

    target = model if inplace else copy.deepcopy(model)
    aliases = {}
    for name, module in target.named_modules(remove_duplicate=False):
        aliases.setdefault(id(module), []).append(name)
    excluded_ids = {key for key, names in aliases.items() if any(_covers(excluded, n) for n in names)}
    selected_ids = {
        key for key, names in aliases.items()
        if key not in excluded_ids
        and all(included is None or _covers(included, n) for n in names)
    }
    internal_ids = {
        id(child)
        for module in target.modules() if isinstance(module, _ANALOG + _TRAINABLE)
        for child in module.modules() if child is not module
    }
    for name, module in target.named_modules():
        if isinstance(module, AnalogMatrix) and module.simulator.device != simulator.device:
            raise ValueError(f"{name}: existing analog matrices are bound to their simulator device")
        if id(module) in internal_ids or id(module) not in selected_ids:
            continue
        if isinstance(module, nn.Conv2d) and isinstance(module.padding, str):
            raise ValueError(f"{name}: numeric Conv2d padding is required")
        if isinstance(module, _ANALOG + _TRAINABLE):
            if (training and isinstance(module, _ANALOG)
                    and not getattr(module, "_hardware_aware_training", False)):
                raise ValueError("training conversion requires the original digital layer weights")
            for child in module.modules():
                if isinstance(child, AnalogMatrix) and (
                    child.config != simulator.config or child.simulator.mode != simulator.mode
                ):
                    raise ValueError(f"{name}: reconversion requires matching physical config and mode")
    target.to(simulator.device)
    replacements = {}

    def bind_cell(result, source, suffix=""):
        for projection, kind in ((result.input, "ih"), (result.hidden, "hh")):
            projection.weight = getattr(source, "weight_" + kind + suffix)
            projection.bias = getattr(source, "bias_" + kind + suffix, None)
            result.register_parameter("weight_" + kind, projection.weight)
            result.register_parameter("bias_" + kind, projection.bias)

    def convert(module, name):
        if id(module) in excluded_ids:
            return module
        if isinstance(module, _SUPPORTED + _ANALOG + _TRAINABLE) and id(module) not in selected_ids:
            return module
        if isinstance(module, _TRAINABLE):
            if training:
                module.gradient_mode = gradient_mode
            return module
        if isinstance(module, _ANALOG):
            if training and not getattr(module, "_hardware_aware_training", False):
                raise ValueError("training conversion requires the original digital layer weights")
            if training:
                for child in module.modules():
                    if isinstance(child, _TRAINABLE + (AnalogRNN, AnalogRNNCell, AnalogGRU,
                                                       AnalogGRUCell)):
                        child.gradient_mode = gradient_mode
            return module
        if id(module) in replacements:
            return replacements[id(module)]
        if isinstance(module, nn.Linear):
            if training:
                result = TrainableAnalogLinear(module, simulator, name=name or "linear",
                                               gradient_mode=gradient_mode)
            else:
                result = AnalogLinear(module, simulator, name=name or "linear")
        elif isinstance(module, nn.Conv2d):
            if training:
                result = TrainableAnalogConv2d(module, simulator, name=name or "conv",
                                               gradient_mode=gradient_mode)
            else:
                result = AnalogConv2d(module, simulator, name=name or "conv")
        elif isinstance(module, (nn.RNNCell, nn.GRUCell)):
            gru = isinstance(module, nn.GRUCell)
            cell_type = AnalogGRUCell if gru else AnalogRNNCell
            result = cell_type(module, simulator, training=training,
                               name=name or ("gru_cell" if gru else "rnn_cell"),
                               gradient_mode=gradient_mode)
        elif isinstance(module, (nn.RNN, nn.GRU)):
            gru = isinstance(module, nn.GRU)
            sequence_type = AnalogGRU if gru else AnalogRNN
            result = sequence_type(module, simulator, training=training,
                                   name=name or ("gru" if gru else "rnn"),
                                   gradient_mode=gradient_mode)
        else:
            result = module
            replacements[id(module)] = result
            for attr, child in list(module._modules.items()):
                if child is not None:
                    setattr(module, attr, convert(child, f"{name}.{attr}" if name else attr))
            config = getattr(module, "config", None)
            if (
                getattr(config, "model_type", None) == "llama"
                and getattr(config, "pretraining_tp", 1) > 1
                and any(isinstance(child, (AnalogLinear, TrainableAnalogLinear))
                        for child in module.modules())
            ):
                config.pretraining_tp = 1
        if training and isinstance(result, _TRAINABLE):
            result.weight, result.bias = module.weight, module.bias
        elif training and isinstance(result, (AnalogRNNCell, AnalogGRUCell)):
            bind_cell(result, module)
        elif training and isinstance(result, (AnalogRNN, AnalogGRU)):
            directions = 2 if result.bidirectional else 1
            for index, cell in enumerate(result.cells):
                suffix = f"_l{index // directions}" + ("_reverse" if index % directions else "")
                bind_cell(cell, module, suffix)
                for attr in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                    result.register_parameter(attr + suffix, getattr(cell, attr))
        replacements[id(module)] = result
        return result

    converted = convert(target, "")
    if training:
        return converted.train()
    return converted.eval().requires_grad_(False)


def reset_read_events(model, event=0):
    """Replay a read event across every programmed matrix, including HAT layers."""
    for module in model.modules():
        if isinstance(module, AnalogMatrix):
            module.reset_read(event)
