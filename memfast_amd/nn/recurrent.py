"""Elman RNN and GRU with analog input and hidden projections (memfast/nn/recurrent.py).

A cell owns two programmed matrices, the input and the hidden projection, with
PyTorch's separate biases; gates and nonlinearities are digital.  Sequences run
stacked layers, both directions, dropout between layers, an explicit initial state and
unbatched input (PackedSequence is not supported).  Each timestep reads both
projections, so a T-step sequence makes 2*T analog reads per layer and direction, and
every read advances its matrix's read event as in the reference.

Two ways of issuing those reads give the same results with fewer host round trips:

* when an input read cannot depend on its read event (no read or voltage variation),
  its input scales are per row and T*B rows select the same kernel as B rows, the T
  input reads of a direction equal one read of all T*B rows; that read is made once
  and the matrix's read event still advances by T;
* the hidden reads of a direction then queue back to back, each OR-ing its error bits
  into one device status word that is read once at the end.  A GRU whose hidden read
  runs on an MFMA kernel issues all its steps (quantize the state, read, add the bias,
  gates) from one native call, ``hip.gru_sequence``; other cells queue them from
  Python.  A clear word means every step read what a checked read returns; otherwise
  the hidden read count is restored and the direction runs again with a check per
  step, which raises or retries in FP64 at the step where the reference does.

Both apply only to inference (no hardware-aware gradients wanted) and only where no
module hooks are registered on the cell or its projections, since they call the
projections' read methods directly.
"""

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.modules import module as _module_globals

from .. import hip
from .linear import AnalogLinear
from .training import TrainableAnalogLinear, _SurrogateGradient, _validate_gradient_mode

_EVENT_LIMIT = 1 << 63
_HOOK_TABLES = ("_forward_hooks", "_forward_pre_hooks", "_backward_hooks", "_backward_pre_hooks")


def _projection(weight, bias, simulator, name, training, gradient_mode):
    """An analog [out, in] projection of ``weight`` and ``bias`` (trainable when
    ``training``): the layers take an nn.Linear source, given here on the meta device
    with the recurrent layer's own Parameters."""
    source = nn.Linear(weight.shape[1], weight.shape[0], bias=bias is not None, device="meta")
    source.weight, source.bias = weight, bias
    if training:
        return TrainableAnalogLinear(source, simulator, name=name, gradient_mode=gradient_mode)
    return AnalogLinear(source, simulator, name=name)


def _initial_hidden(x, hx, input_size, hidden_size, kind):
    """The cell's hidden state: zeros, or ``hx`` checked against the input."""
    valid_input = (torch.is_tensor(x) and x.ndim in (1, 2) and x.shape[-1] == input_size
                   and x.is_floating_point())
    if not valid_input:
        raise ValueError(f"{kind} input must be floating [input_size] or [batch, input_size]")
    shape = (*x.shape[:-1], hidden_size)
    if hx is None:
        return x.new_zeros(shape)
    if not (torch.is_tensor(hx) and hx.shape == shape and hx.device == x.device
            and hx.dtype == x.dtype):
        raise ValueError("hidden state must match the input batch, device, and dtype")
    return hx


def _hooked(*modules):
    """Whether calling these modules would run any forward or backward hook."""
    if any(getattr(_module_globals, f"_global{table}", None) for table in _HOOK_TABLES):
        return True
    return any(getattr(module, table, None) for module in modules for table in _HOOK_TABLES)


class _AnalogCell(nn.Module):
    """A recurrent cell over two analog projections; subclasses give the digital
    combination of the projections (``_analog``) and its FP32 surrogate."""

    source_type, kind, default_name = None, "", ""

    def __init__(self, source, simulator, *, training=False, name=None,
                 gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, self.source_type):
            raise TypeError(f"source must be torch.nn.{self.kind}")
        name = self.default_name if name is None else name
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self._hardware_aware_training = training
        self.input_size, self.hidden_size, self.bias = (source.input_size, source.hidden_size,
                                                        source.bias)
        self._copy_options(source)
        for role, kind in (("input", "ih"), ("hidden", "hh")):
            setattr(self, role, _projection(getattr(source, f"weight_{kind}"),
                                            getattr(source, f"bias_{kind}"), simulator,
                                            f"{name}.{role}", training, gradient_mode))
        self.train(source.training)

    def _copy_options(self, source):
        pass

    def forward(self, x, hx=None):
        hx = _initial_hidden(x, hx, self.input_size, self.hidden_size, self.kind)
        inputs, hidden = self.input(x), self.hidden(hx)
        analog = self._analog(inputs.detach(), hidden.detach(), hx.detach())
        if self._hardware_aware_training and torch.is_grad_enabled():
            return _SurrogateGradient.apply(analog, self._surrogate(inputs, hidden, hx))
        return analog

    def _step(self, inputs, hx, status=None):
        """One inference step from this step's input projection ``inputs``.  With
        ``status`` the hidden read defers its checks to that word."""
        hidden = self.hidden(hx) if status is None else self.hidden._forward_deferred(hx, status)
        return self._analog(inputs, hidden, hx)


class AnalogRNNCell(_AnalogCell):
    """``nn.RNNCell``: activation(W_ih x + b_ih + W_hh h + b_hh), tanh or ReLU."""

    source_type, kind, default_name = nn.RNNCell, "RNNCell", "rnn_cell"

    def __init__(self, source, simulator, *, training=False, name="rnn_cell",
                 gradient_mode="quantized"):
        super().__init__(source, simulator, training=training, name=name,
                         gradient_mode=gradient_mode)

    def _copy_options(self, source):
        self.nonlinearity = source.nonlinearity

    def _activation(self, value):
        return torch.tanh(value) if self.nonlinearity == "tanh" else F.relu(value)

    def _analog(self, inputs, hidden, hx):
        return self._activation(inputs + hidden)

    def _surrogate(self, inputs, hidden, hx):
        return self._activation((inputs + hidden).float())


class AnalogGRUCell(_AnalogCell):
    """``nn.GRUCell``: reset, update and new gates in PyTorch's order and equations (the
    reset gate scales the whole hidden candidate projection, bias included)."""

    source_type, kind, default_name = nn.GRUCell, "GRUCell", "gru_cell"

    def __init__(self, source, simulator, *, training=False, name="gru_cell",
                 gradient_mode="quantized"):
        super().__init__(source, simulator, training=training, name=name,
                         gradient_mode=gradient_mode)

    @staticmethod
    def _gates(inputs, hidden, hx):
        width = inputs.shape[-1] // 3
        # Reset and update gates in one elementwise pass over both thirds: the same
        # per-element operations as sigmoid(i_r + h_r) and sigmoid(i_z + h_z).
        gates = torch.sigmoid(inputs[..., :2 * width] + hidden[..., :2 * width])
        reset, update = gates[..., :width], gates[..., width:]
        candidate = torch.tanh(inputs[..., 2 * width:] + reset * hidden[..., 2 * width:])
        return (1 - update) * candidate + update * hx

    def _analog(self, inputs, hidden, hx):
        fused = (inputs.ndim == 2 and inputs.dtype == hidden.dtype == hx.dtype == torch.float32
                 and inputs.stride(1) == hidden.stride(1) == hx.stride(1) == 1)
        # FP32 gates as one kernel, rounding as the elementwise operations of _gates.
        return hip.gru_gates(inputs, hidden, hx) if fused else self._gates(inputs, hidden, hx)

    def _surrogate(self, inputs, hidden, hx):
        return self._gates(inputs.float(), hidden.float(), hx.float())


def _batchable_inputs(projection, steps, batch):
    """Whether ``steps`` input reads of ``batch`` rows equal one read of all rows."""
    if type(projection) is not AnalogLinear or steps < 2:
        return False
    config = projection.config
    effects = config.nonidealities
    rowwise_scales = projection.input_scale is not None or config.input_quant_gran[0] == 1
    if (projection.simulator.mode != "default" or not rowwise_scales or effects.read_variation
            or effects.voltage_variation or projection._event + steps >= _EVENT_LIMIT):
        return False
    arrays = -(-projection.in_features // config.array_size[0])
    return (hip.mm_kernel(config, steps * batch, arrays, projection.p)
            == hip.mm_kernel(config, batch, arrays, projection.p))


class _AnalogRecurrent(nn.Module):
    """Sequence traversal shared by AnalogRNN and AnalogGRU."""

    source_type = cell_type = analog_cell_type = None
    kind = ""
    _OPTIONS = ("input_size", "hidden_size", "num_layers", "bias", "batch_first", "dropout",
                "bidirectional")

    def __init__(self, source, simulator, *, training=False, name=None, gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, self.source_type):
            raise TypeError(f"source must be torch.nn.{self.kind}")
        name = self.kind.lower() if name is None else name
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self._hardware_aware_training = training
        for option in self._OPTIONS:
            setattr(self, option, getattr(source, option))
        if isinstance(source, nn.RNN):
            self.nonlinearity = source.nonlinearity
        self.cells = nn.ModuleList(
            self.analog_cell_type(self._layer_cell(source, layer, direction), simulator,
                                  training=training, name=f"{name}.layer{layer}.direction{direction}",
                                  gradient_mode=gradient_mode)
            for layer in range(self.num_layers) for direction in range(self._directions)
        )
        self.train(source.training)

    @property
    def _directions(self):
        return 2 if self.bidirectional else 1

    def _layer_cell(self, source, layer, direction):
        """A torch cell (on the meta device) holding ``source``'s Parameters of one layer
        and direction (PyTorch's ``_l{layer}[_reverse]`` names)."""
        width = self.input_size if layer == 0 else self.hidden_size * self._directions
        options = {"nonlinearity": self.nonlinearity} if isinstance(source, nn.RNN) else {}
        cell = self.cell_type(width, self.hidden_size, bias=self.bias, device="meta", **options)
        suffix = f"_l{layer}" + ("_reverse" if direction else "")
        for parameter in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
            setattr(cell, parameter, getattr(source, parameter + suffix, None))
        return cell

    def _sequence_and_state(self, x, hx):
        """([T, B, input] time-major sequence, [layers*directions, B, hidden] state,
        whether the input was unbatched), with the reference's checks."""
        valid = (torch.is_tensor(x) and x.ndim in (2, 3) and x.shape[-1] == self.input_size
                 and x.is_floating_point())
        if not valid:
            raise ValueError(
                f"{self.kind} input must be a floating dense sequence with matching input_size")
        unbatched = x.ndim == 2
        if unbatched:
            sequence = x.unsqueeze(1)
        else:
            sequence = x.transpose(0, 1) if self.batch_first else x
        if sequence.shape[0] == 0:
            raise ValueError(f"{self.kind} sequence must contain at least one timestep")
        shape = (self.num_layers * self._directions, sequence.shape[1], self.hidden_size)
        if hx is None:
            return sequence, x.new_zeros(shape), unbatched
        expected = (shape[0], shape[2]) if unbatched else shape
        if not (torch.is_tensor(hx) and hx.shape == expected and hx.device == x.device
                and hx.dtype == x.dtype):
            raise ValueError("hidden state must match layers, directions, batch, device, and dtype")
        return sequence, hx.unsqueeze(1) if unbatched else hx, unbatched

    def forward(self, x, hx=None):
        sequence, state, unbatched = self._sequence_and_state(x, hx)
        finals = []
        for layer in range(self.num_layers):
            outputs = []
            for direction in range(self._directions):
                index = layer * self._directions + direction
                states, final = self._traverse(self.cells[index], sequence, state[index],
                                               reverse=bool(direction))
                outputs.append(states)
                finals.append(final)
            sequence = outputs[0] if len(outputs) == 1 else torch.cat(outputs, dim=-1)
            if self.dropout and layer + 1 < self.num_layers:
                sequence = self._dropout(sequence)
        hidden = torch.stack(finals)
        if unbatched:
            return sequence.squeeze(1), hidden.squeeze(1)
        return (sequence.transpose(0, 1) if self.batch_first else sequence), hidden

    def _dropout(self, sequence):
        """Dropout between layers; under hardware-aware training the analog values and
        their FP32 surrogate share one mask."""
        if not (self._hardware_aware_training and torch.is_grad_enabled()):
            return F.dropout(sequence, p=self.dropout, training=self.training)
        mask = F.dropout(torch.ones_like(sequence), p=self.dropout, training=self.training)
        return _SurrogateGradient.apply(sequence.detach() * mask, sequence.float() * mask.float())

    def _traverse(self, cell, sequence, hidden, *, reverse):
        """([T, B, hidden] states in time order, final state) of one direction."""
        order = list(range(sequence.shape[0]))
        if reverse:
            order.reverse()
        projected = self._projected_inputs(cell, sequence)
        if projected is not None:
            return self._steps(cell, projected, order, hidden)
        states = []
        for step in order:
            hidden = cell(sequence[step], hidden)
            states.append(hidden)
        return _in_time_order(states, order), hidden

    def _projected_inputs(self, cell, sequence):
        """Every step's input projection from one read, or None to read per step."""
        steps = sequence.shape[0]
        batch = sequence[0].numel() // sequence.shape[-1]
        usable = (batch > 0 and not (self._hardware_aware_training and torch.is_grad_enabled())
                  and not _hooked(cell, cell.input, cell.hidden)
                  and _batchable_inputs(cell.input, steps, batch))
        if not usable:
            return None
        matrix = cell.input
        start = matrix._event
        try:
            with torch.no_grad():
                projected = matrix._forward(sequence, retry=False)
        except (ValueError, FloatingPointError):
            projected = None
        if projected is None:
            # The per-step reads raise, or retry in FP64, where the reference does.
            matrix._event = start
            return None
        matrix._event = start + steps
        return projected

    @staticmethod
    def _steps(cell, projected, order, hidden):
        """([T, B, H] states in time order, final state) of one direction from precomputed
        input projections.  A GRU whose hidden read allows it runs every step in one native
        call (``hip.gru_sequence``) with the checks deferred to one status word; other
        cells queue their steps from Python with the same deferral; if that word is set,
        the steps run again with a check per step.

        If a step raises, the input projection's read count is set to what per-step
        reading would have left (one more than the steps completed before it); the
        hidden projection's count is what its reads left."""
        input_start = cell.input._event - len(order)
        if _native_eligible(cell, projected, hidden, len(order)):
            try:
                result = _native_steps(cell, projected, order, hidden)
            except Exception:
                cell.input._event = input_start + 1
                raise
            if result is not None:
                return result
        attempts = ((True, False) if cell.hidden._deferrable(hidden, len(order)) else (False,))
        for deferred in attempts:
            hidden_start = cell.hidden._event
            status = hip.status_word(hidden.device) if deferred else None
            state, states, done = hidden, [], 0
            try:
                with torch.no_grad():
                    for step in order:
                        state = cell._step(projected[step], state, status)
                        states.append(state)
                        done += 1
            except Exception:
                cell.input._event = input_start + done + 1
                raise
            if status is None or int(status.item()) == 0:
                return _in_time_order(states, order), state
            cell.hidden._event = hidden_start
        raise AssertionError("the checked attempt always returns or raises")


def _in_time_order(states, order):
    """Stack states collected in traversal ``order`` as [T, ...] in time order."""
    if order and order[0] > order[-1]:
        states = states[::-1]
    return torch.stack(states)


def _native_eligible(cell, projected, hidden, steps):
    """Whether a GRU direction can run in one ``hip.gru_sequence`` call: an inference
    cell whose hidden read is deferrable FP32 with dynamic input scales on an MFMA kernel."""
    if not isinstance(cell, AnalogGRUCell):
        return False
    matrix = cell.hidden
    if (type(matrix) is not AnalogLinear or matrix.input_scale is not None
            or projected.dtype != torch.float32 or not matrix._deferrable(hidden, steps)):
        return False
    arrays = -(-matrix.in_features // matrix.config.array_size[0])
    return hip.mm_kernel(matrix.config, hidden.shape[0], arrays, matrix.p) in (1, 2)


def _native_steps(cell, projected, order, hidden):
    """The steps of ``_AnalogRecurrent._steps`` as one native call: ([T, B, H] states,
    final state), or None (read count unchanged) when the status word is set."""
    matrix = cell.hidden
    config = matrix.config
    batch = hidden.shape[0]
    arrays = -(-matrix.in_features // config.array_size[0])
    codes_t = matrix._column_codes()
    source = None
    if hip.mm_kernel(config, batch, arrays, matrix.p) == 2 and hip.terms_event_independent(config):
        workspace, reuse, source = matrix._terms_workspace(batch, arrays, hidden.device, codes_t)
    else:
        workspace = hip._workspace(config, batch, arrays, matrix.p, hidden.device)
        reuse = False
    status = hip.status_word(hidden.device)
    bias = None if matrix.bias is None else matrix.bias.contiguous()
    columns = matrix.p * config.array_size[1]
    states = hip.gru_sequence(config, projected.contiguous(), hidden.contiguous(), matrix.packed,
                              codes_t, matrix.weight_scale.reshape(-1, columns), bias,
                              matrix.seed, matrix._event, reverse=order[0] > order[-1],
                              status=status, workspace=workspace, reuse_terms=reuse)
    if source is not None:
        matrix._terms_source = source
    if int(status.item()):
        return None
    matrix._event += len(order)
    return states, states[order[-1]]


class AnalogRNN(_AnalogRecurrent):
    """``nn.RNN`` (tanh or ReLU, stacked, bidirectional, unbatched) over analog cells."""

    source_type, cell_type, analog_cell_type, kind = nn.RNN, nn.RNNCell, AnalogRNNCell, "RNN"


class AnalogGRU(_AnalogRecurrent):
    """``nn.GRU`` with PyTorch's gate equations over analog cells."""

    source_type, cell_type, analog_cell_type, kind = nn.GRU, nn.GRUCell, AnalogGRUCell, "GRU"
