"""Helpers for noisy-device parity tests: the GPU slice totals behind a product and the
oracle's totals and outputs for the same codes, seeds and read events.

A read with device noise is compared in two parts.  Its slice totals come from
the same kernel the product uses (``hip.mm_kernel``), in its totals mode; they
are deterministic (counter-based RNG), so they are the totals behind the
product.  ``oracle.flips.check_noisy`` then counts the flipped codes and checks
each output against the oracle's.
"""

import torch

from memfast_amd import hip
from oracle import flips, oracle


def say(*args):
    print("[parity]", *args, flush=True)


def gpu_totals(q, packed, cfg, seed, event, *, codes_t=None, conductance=None):
    """Slice totals [N, G, p, C] (FP64) of the kernel ``hip.mm`` runs for these operands.

    q, packed: device codes [N, m, R] and [m, p, R, C].  ``conductance``
    (optional) injects FP32 conductances [m, p, W, R, C] into the MFMA kernels
    (the general kernel takes [planes, m, p, W, R, C])."""
    n, m, _ = q.shape
    p = packed.shape[1]
    kernel = hip.mm_kernel(cfg, n, m, p)
    if kernel == 2:
        if codes_t is None:
            codes_t = hip.kernel_codes(packed, cfg)
        return hip.mm_totals(q, codes_t, cfg, seed, event, conductance=conductance).double()
    if kernel == 3:
        return hip.mm_totals_wide(q, packed, cfg, seed, event, conductance=conductance).double()
    assert kernel == 0, "ideal devices are compared bit for bit, not through totals"
    return hip.partial(q, packed, cfg, None, seed, event, 0, p, conductance=conductance).double()


def oracle_totals(q, packed, cfg, seed, event, *, tiles=None, conductance=None):
    """Oracle slice totals [N, G, p, C] for the tiles in ``tiles`` (default all); other
    tiles are left at zero.  Chunks of two tiles, as memfast/simulator.py:575-577."""
    n, m, _ = q.shape
    p = packed.shape[1]
    first, last = (0, p) if tiles is None else tiles
    totals = torch.zeros((n, m * oracle.reads_per_array(cfg), p, cfg.array_size[1]),
                         dtype=torch.float64)
    for begin in range(first, last, 2):
        end = min(begin + 2, last)
        injected = None if conductance is None else conductance[:, begin:end]
        totals[:, :, begin:end] = oracle.partial(q, packed, cfg, seed, event, begin, end,
                                                 conductance=injected).double()
    return totals


def check_read(cfg, got, q, xscale, packed, wscale, seed, event, got_totals, *, tiles=None,
               bias=None, label=""):
    """Flip-aware parity of one read's output ``got`` [N, O'] against the oracle.

    ``q``/``xscale``/``packed``/``wscale`` are the oracle's (CPU) tiles of the
    same operands; ``got_totals`` the GPU totals [N, G, p, C].  With ``tiles``
    only those tiles' columns of ``got`` (already sliced by the caller) are
    checked.  Returns the flip report."""
    p, c = packed.shape[1], cfg.array_size[1]
    ref_totals = oracle_totals(q, packed, cfg, seed, event, tiles=tiles)
    first, last = (0, p) if tiles is None else tiles
    if tiles is None:
        expected = oracle.execute(q, xscale, packed, wscale, cfg, seed, event, got.shape[1],
                                  bias=bias, totals=ref_totals)
    else:
        expected = oracle.execute(q, xscale, packed, wscale, cfg, seed, event, p * c,
                                  totals=ref_totals, tiles=tiles)
        if bias is not None:
            expected = expected + bias[first * c:last * c]
    # The product is returned in the operands' dtype (memfast/simulator.py:635-646): compare
    # in that dtype, so clean outputs are bit-identical.
    expected = expected.to(got.dtype)
    width = expected.shape[1]
    sub_got = got_totals.cpu()[:, :, first:last]
    sub_ref = ref_totals[:, :, first:last]
    ws = wscale.reshape(wscale.shape[0], -1)[:, first * c:last * c]
    report = flips.check_noisy(cfg, got.cpu()[:, :width], expected, sub_got, sub_ref,
                               xscale=xscale, wscale=ws, label=label)
    say(report)
    return report


def gru_step_parity(cell, source, x, output, device, *, label="gru"):
    """Step-by-step parity of a one-layer, one-direction AnalogGRU sequence ``output``
    [T, B, H] over inputs ``x`` [T, B, I] (CPU), converted from ``source`` (nn.GRU).

    For each step t, the cell's two projections are read again at read event t
    from the sequence's own hidden state.  Asserts that the sequence's step-t
    output is PyTorch's gate equations over those reads, bit for bit on the GPU
    (``hip.gru_gates``) and within transcendental rounding against torch's CPU
    ops; and that each read matches the oracle (``check_product``) as
    memfast/nn/recurrent.py:101-116 composes them."""
    h = torch.zeros(x.shape[1], cell.hidden_size, device=device)
    for t in range(x.shape[0]):
        cell.input.reset_read(t)
        cell.hidden.reset_read(t)
        inputs = cell.input(x[t].to(device))
        hid = cell.hidden(h)
        gates = hip.gru_gates(inputs, hid, h)
        assert torch.equal(output[t].view(torch.int32), gates.view(torch.int32)), (label, t)
        check_product(cell.input.config, inputs, x[t], source.weight_ih_l0.T, device,
                      name=cell.input.name, event=t, bias=source.bias_ih_l0,
                      label=f"{label} step {t} input")
        check_product(cell.hidden.config, hid, h, source.weight_hh_l0.T, device,
                      name=cell.hidden.name, event=t, bias=source.bias_hh_l0,
                      label=f"{label} step {t} hidden")
        ir, iz, inn = inputs.cpu().chunk(3, dim=-1)
        hr, hz, hn = hid.cpu().chunk(3, dim=-1)
        reset = torch.sigmoid(ir + hr)
        update = torch.sigmoid(iz + hz)
        expected = (1 - update) * torch.tanh(inn + reset * hn) + update * h.cpu()
        torch.testing.assert_close(output[t].cpu(), expected, rtol=1e-5, atol=1e-6)
        h = output[t]


def check_product(cfg, got, a, b, device, *, name="matrix.0", event=0, bias=None, label=""):
    """``got`` is a read of A [..., K] through B [K, O] programmed as ``name`` at read
    ``event`` (optionally plus ``bias``).  Ideal devices: bit for bit against the oracle.
    Device noise: flip-aware against the oracle (its own conductance samples)."""
    a = a.detach().cpu().reshape(-1, b.shape[0])
    q, xs = oracle.input_tiles(a, cfg)
    packed, ws = oracle.weight_tiles(b.detach().cpu().T, cfg)
    seed = oracle.name_seed(cfg.seed, name)
    got = got.detach().reshape(a.shape[0], -1)
    bias = None if bias is None else bias.detach().cpu().to(got.dtype)
    if cfg.nonidealities.ideal:
        expected = oracle.execute(q, xs, packed, ws, cfg, seed, event, b.shape[1], bias=bias)
        expected = expected.to(got.dtype)
        view = torch.int32 if got.dtype == torch.float32 else torch.int64
        assert torch.equal(got.cpu().view(view), expected.view(view)), (
            label, (got.cpu().double() - expected.double()).abs().max())
        return None
    totals = gpu_totals(q.to(device), packed.to(device), cfg, seed, event)
    return check_read(cfg, got, q, xs, packed, ws, seed, event, totals, bias=bias, label=label)
