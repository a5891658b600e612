"""Elman RNN and GRU recurrences with analog input and hidden projections.

Restates memfast/nn/recurrent.py.  Each cell owns two programmed matrices
(input and hidden projection, biases kept separate as in PyTorch); gates and
nonlinearities stay digital.  Sequences support stacked layers, both
directions, inter-layer dropout, explicit initial state and unbatched input;
PackedSequence is not supported.  Every timestep reads both projections, so
a T-step sequence issues 2*T analog products per layer and direction.

When a read's result cannot depend on its read event (no read or voltage
variation) and input quantization groups do not span rows, the T input
projections of a sequence equal one product over all T*B rows: that product
is issued once and the input matrix's event counter still advances by T.
"""

import torch
from torch import nn
from torch.nn import functional as F

from .. import hip
from .linear import AnalogLinear
from .training import TrainableAnalogLinear, _SurrogateGradient, _validate_gradient_mode


def _batchable_inputs(projection, steps, batch):
    """Whether the T per-step reads of ``projection`` (``batch`` rows each) equal one
    read over all rows: same kernel, no event-dependent noise, per-row input scales."""
    if type(projection) is not AnalogLinear or steps < 2:
        return False
    config = projection.config
    effects = config.nonidealities
    per_row = projection.input_scale is not None or config.input_quant_gran[0] == 1
    if not (projection.simulator.mode == "default" and per_row
            and not effects.read_variation and not effects.voltage_variation
            and projection._event + steps < 2**63):
        return False
    m = -(-projection.in_features // config.array_size[0])
    return (hip.mm_kernel(config, steps * batch, m, projection.p)
            == hip.mm_kernel(config, batch, m, projection.p))


def _projection(weight, bias, simulator, name, training, gradient_mode):
    source = nn.Linear(weight.shape[1], weight.shape[0], bias=bias is not None, device="meta")
    source.weight, source.bias = weight, bias
    if training:
        return TrainableAnalogLinear(source, simulator, name=name, gradient_mode=gradient_mode)
    return AnalogLinear(source, simulator, name=name)


def _initial_hidden(x, hx, input_size, hidden_size, kind):
    if (
        not torch.is_tensor(x)
        or x.ndim not in (1, 2)
        or x.shape[-1] != input_size
        or not x.is_floating_point()
    ):
        raise ValueError(f"{kind} input must be floating [input_size] or [batch, input_size]")
    shape = (*x.shape[:-1], hidden_size)
    if hx is None:
        return x.new_zeros(shape)
    if not torch.is_tensor(hx) or hx.shape != shape or hx.device != x.device or hx.dtype != x.dtype:
        raise ValueError("hidden state must match the input batch, device, and dtype")
    return hx


class AnalogRNNCell(nn.Module):
    """``nn.RNNCell`` with analog input and hidden projections."""

    def __init__(self, source, simulator, *, training=False, name="rnn_cell",
                 gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.RNNCell):
            raise TypeError("source must be torch.nn.RNNCell")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self._hardware_aware_training = training
        self.input_size, self.hidden_size = source.input_size, source.hidden_size
        self.nonlinearity, self.bias = source.nonlinearity, source.bias
        self.input = _projection(source.weight_ih, source.bias_ih, simulator, f"{name}.input",
                                 training, gradient_mode)
        self.hidden = _projection(source.weight_hh, source.bias_hh, simulator, f"{name}.hidden",
                                  training, gradient_mode)
        self.train(source.training)

    def forward(self, x, hx=None):
        hx = _initial_hidden(x, hx, self.input_size, self.hidden_size, "RNNCell")
        value = self.input(x) + self.hidden(hx)
        activation = torch.tanh if self.nonlinearity == "tanh" else F.relu
        analog = activation(value.detach())
        if self._hardware_aware_training and torch.is_grad_enabled():
            return _SurrogateGradient.apply(analog, activation(value.float()))
        return analog

    def _step(self, inputs, hx, status=None):
        """One inference step given this step's input projection (``status``: the
        deferred status word of ``_AnalogRecurrent._deferred_steps``)."""
        activation = torch.tanh if self.nonlinearity == "tanh" else F.relu
        hidden = self.hidden(hx) if status is None else self.hidden._forward_deferred(hx, status)
        return activation(inputs + hidden)


class AnalogGRUCell(nn.Module):
    """``nn.GRUCell`` gates (reset, update, new) over analog projections."""

    def __init__(self, source, simulator, *, training=False, name="gru_cell",
                 gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, nn.GRUCell):
            raise TypeError("source must be torch.nn.GRUCell")
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self._hardware_aware_training = training
        self.input_size, self.hidden_size = source.input_size, source.hidden_size
        self.bias = source.bias
        self.input = _projection(source.weight_ih, source.bias_ih, simulator, f"{name}.input",
                                 training, gradient_mode)
        self.hidden = _projection(source.weight_hh, source.bias_hh, simulator, f"{name}.hidden",
                                  training, gradient_mode)
        self.train(source.training)

    @staticmethod
    def _gates(inputs, hidden, hx):
        # reset and update gates in one elementwise pass over both chunks (the same
        # per-element operations as sigmoid(ir + hr) and sigmoid(iz + hz)).
        width = inputs.shape[-1] // 3
        gates = torch.sigmoid(inputs[..., :2 * width] + hidden[..., :2 * width])
        reset, update = gates[..., :width], gates[..., width:]
        candidate = torch.tanh(inputs[..., 2 * width:] + reset * hidden[..., 2 * width:])
        return (1 - update) * candidate + update * hx

    def forward(self, x, hx=None):
        hx = _initial_hidden(x, hx, self.input_size, self.hidden_size, "GRUCell")
        inputs, hidden = self.input(x), self.hidden(hx)
        analog = self._gates(inputs.detach(), hidden.detach(), hx.detach())
        if self._hardware_aware_training and torch.is_grad_enabled():
            surrogate = self._gates(inputs.float(), hidden.float(), hx.float())
            return _SurrogateGradient.apply(analog, surrogate)
        return analog

    def _step(self, inputs, hx, status=None):
        """One inference step given this step's input projection.  FP32 gates run as one
        kernel with the same roundings as the elementwise ops of ``_gates``.  ``status``:
        the deferred status word of ``_AnalogRecurrent._deferred_steps``."""
        hidden = self.hidden(hx) if status is None else self.hidden._forward_deferred(hx, status)
        if (inputs.ndim == 2 and inputs.dtype == hidden.dtype == hx.dtype == torch.float32
                and inputs.stride(1) == hidden.stride(1) == hx.stride(1) == 1):
            return hip.gru_gates(inputs, hidden, hx)
        return self._gates(inputs, hidden, hx)


class _AnalogRecurrent(nn.Module):
    """Dense sequence traversal shared by AnalogRNN and AnalogGRU."""

    source_type = cell_type = analog_cell_type = None
    kind = ""

    def __init__(self, source, simulator, *, training=False, name=None, gradient_mode="quantized"):
        super().__init__()
        if not isinstance(source, self.source_type):
            raise TypeError(f"source must be torch.nn.{self.kind}")
        name = self.kind.lower() if name is None else name
        self.gradient_mode = _validate_gradient_mode(gradient_mode)
        self._hardware_aware_training = training
        for attr in ("input_size", "hidden_size", "num_layers", "bias", "batch_first", "dropout",
                     "bidirectional"):
            setattr(self, attr, getattr(source, attr))
        if isinstance(source, nn.RNN):
            self.nonlinearity = source.nonlinearity
        self.cells = nn.ModuleList()
        directions = 2 if self.bidirectional else 1
        for layer in range(self.num_layers):
            width = self.input_size if layer == 0 else self.hidden_size * directions
            for direction in range(directions):
                suffix = f"_l{layer}" + ("_reverse" if direction else "")
                extra = {"nonlinearity": self.nonlinearity} if isinstance(source, nn.RNN) else {}
                cell = self.cell_type(width, self.hidden_size, bias=self.bias, device="meta", **extra)
                for attr in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                    setattr(cell, attr, getattr(source, attr + suffix, None))
                self.cells.append(self.analog_cell_type(
                    cell, simulator, training=training,
                    name=f"{name}.layer{layer}.direction{direction}", gradient_mode=gradient_mode,
                ))
        self.train(source.training)

    def forward(self, x, hx=None):
        if (
            not torch.is_tensor(x)
            or x.ndim not in (2, 3)
            or x.shape[-1] != self.input_size
            or not x.is_floating_point()
        ):
            raise ValueError(
                f"{self.kind} input must be a floating dense sequence with matching input_size"
            )
        unbatched = x.ndim == 2
        sequence = x.unsqueeze(1) if unbatched else (x.transpose(0, 1) if self.batch_first else x)
        if sequence.shape[0] == 0:
            raise ValueError(f"{self.kind} sequence must contain at least one timestep")
        directions = 2 if self.bidirectional else 1
        shape = (self.num_layers * directions, sequence.shape[1], self.hidden_size)
        expected = (shape[0], shape[2]) if unbatched else shape
        if hx is None:
            state = x.new_zeros(shape)
        else:
            if (not torch.is_tensor(hx) or hx.shape != expected or hx.device != x.device
                    or hx.dtype != x.dtype):
                raise ValueError("hidden state must match layers, directions, batch, device, and dtype")
            state = hx.unsqueeze(1) if unbatched else hx
        final = []
        for layer in range(self.num_layers):
            outputs = []
            for direction in range(directions):
                index = layer * directions + direction
                hidden = state[index]
                steps = range(sequence.shape[0])
                if direction:
                    steps = reversed(steps)
                steps = list(steps)
                values = []
                cell = self.cells[index]
                # Read count of the input projection before this traversal (the
                # batched projection below advances it by the number of steps).
                start = cell.input._event
                projected = self._projected_inputs(cell, sequence)
                if projected is None:
                    for step in steps:
                        hidden = cell(sequence[step], hidden)
                        values.append(hidden)
                elif (deferred := self._deferred_steps(cell, projected, steps, hidden)):
                    values, hidden = deferred
                else:
                    matrix = cell.input
                    for count, step in enumerate(steps):
                        try:
                            hidden = cell._step(projected[step], hidden)
                        except Exception:
                            # The reference would have read the input projection
                            # count + 1 times when this step's hidden read failed.
                            matrix._event = start + count + 1
                            raise
                        values.append(hidden)
                if direction:
                    values.reverse()
                outputs.append(torch.stack(values))
                final.append(hidden)
            sequence = torch.cat(outputs, dim=-1) if directions == 2 else outputs[0]
            if self.dropout and layer + 1 < self.num_layers:
                if self._hardware_aware_training and torch.is_grad_enabled():
                    mask = F.dropout(torch.ones_like(sequence), p=self.dropout, training=self.training)
                    sequence = _SurrogateGradient.apply(sequence.detach() * mask,
                                                        sequence.float() * mask.float())
                else:
                    sequence = F.dropout(sequence, p=self.dropout, training=self.training)
        hidden = torch.stack(final)
        if unbatched:
            return sequence.squeeze(1), hidden.squeeze(1)
        output = sequence.transpose(0, 1) if self.batch_first else sequence
        return output, hidden


    @staticmethod
    def _deferred_steps(cell, projected, steps, hidden):
        """The step loop with one status read for the whole traversal, or None.

        Each hidden read ORs its status bits into one word (``_forward_deferred``),
        so the reads queue without a host wait per step.  A clear word at the end
        means every step read what a per-step read returns and nothing raised.
        Otherwise the hidden projection's read count is restored and None makes
        the caller redo the loop with a status read per step, which raises or
        retries at the step where per-step reading does."""
        matrix = cell.hidden
        if not matrix._deferrable(hidden, len(steps)):
            return None
        start = matrix._event
        status = hip.status_word(hidden.device)
        values = []
        try:
            with torch.no_grad():   # as forward() of the hidden projection
                for step in steps:
                    hidden = cell._step(projected[step], hidden, status)
                    values.append(hidden)
            clear = int(status.item()) == 0
        except Exception:
            matrix._event = start
            raise
        if not clear:
            matrix._event = start
            return None
        return values, hidden

    def _projected_inputs(self, cell, sequence):
        """All steps' input projections from one read, or None to read per step."""
        steps = sequence.shape[0]
        batch = sequence[0].numel() // sequence.shape[-1]
        if ((self._hardware_aware_training and torch.is_grad_enabled()) or batch == 0
                or not _batchable_inputs(cell.input, steps, batch)):
            return None
        matrix = cell.input
        start = matrix._event
        try:
            with torch.no_grad():
                projected = matrix._forward(sequence, retry=False)
        except (ValueError, FloatingPointError):
            projected = None
        if projected is None:
            # Per-step reads then raise (or retry in FP64) where the reference does.
            matrix._event = start
            return None
        matrix._event = start + steps
        return projected


class AnalogRNN(_AnalogRecurrent):
    """``nn.RNN`` (tanh/ReLU, stacked, bidirectional, unbatched) with analog projections."""

    source_type, cell_type, analog_cell_type, kind = nn.RNN, nn.RNNCell, AnalogRNNCell, "RNN"


class AnalogGRU(_AnalogRecurrent):
    """``nn.GRU`` with PyTorch gate equations over analog projections."""

    source_type, cell_type, analog_cell_type, kind = nn.GRU, nn.GRUCell, AnalogGRUCell, "GRU"
