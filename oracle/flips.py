"""Rounding-flip accounting for noisy-device parity (TEST INFRASTRUCTURE ONLY).

With device noise the GPU's currents are summed in a different FP32 order than
the reference's ``torch.bmm`` (memfast/reference.py:101), so an ADC count whose
argument lies within rounding distance of a half-integer may differ by one.
BASELINE's bar: identical codes except such flips (at most 1e-4 of all codes)
and output relative error <= 1e-5 elsewhere.

The MFMA kernels return slice totals T[n, g, t, c] = sum_aw fa*fw*code_aw
(memfast/reference.py:115), not the individual codes.  A total that differs
from the oracle's is explained here by the fewest single-count code changes
(each pair (a, w) contributes at most one change of +-1, so a difference must
be a sum of distinct +-fa*fw terms).  That count is a lower bound on the
flipped codes and, because two flips inside one total are rare, normally the
exact number.  A difference that no three such changes explain fails the
check outright.

Only ``tests/`` and ``__graft_entry__.smoke()`` import this module.
"""

import itertools

import torch

from .oracle import (adc_maxima, input_layout, precise_currents, read_rows, reads_per_array,
                     weight_layout)


def pair_factors(cfg):
    """Signed fa*fw of every (input slice, weight slice) pair (memfast/config.py:193-201)."""
    return [fa * fw for _, _, fa in input_layout(cfg) for _, _, fw in weight_layout(cfg)]


def _explanations(cfg, depth=3):
    """Map from a total difference to the fewest distinct-pair +-1 code changes making it."""
    factors = pair_factors(cfg)
    best = {0: 0}
    for count in range(1, depth + 1):
        for pairs in itertools.combinations(range(len(factors)), count):
            for signs in itertools.product((1, -1), repeat=count):
                value = sum(s * factors[i] for s, i in zip(signs, pairs))
                best.setdefault(value, count)
    return best


def count_flips(cfg, got_totals, ref_totals):
    """(differing totals, flipped codes lower bound, unexplained totals, mask [N, G, p, C])."""
    diff = got_totals.double().cpu() - ref_totals.double().cpu()
    mask = diff != 0
    values = diff[mask]
    if not values.numel():
        return 0, 0, 0, mask
    table = _explanations(cfg)
    flips = unexplained = 0
    for value, occurrences in zip(*torch.unique(values, return_counts=True)):
        v = float(value)
        need = table.get(int(v)) if v == int(v) else None
        if need is None:
            unexplained += int(occurrences)
        else:
            flips += need * int(occurrences)
    return int(mask.sum()), flips, unexplained, mask


def check_noisy(cfg, got, expected, got_totals, ref_totals, *, xscale=None, wscale=None,
                label=""):
    """Assert BASELINE's noisy-device bar on one product.

    got, expected: outputs [N, O] (GPU, oracle); got_totals, ref_totals: slice
    totals [N, G, p, C] behind them (O <= p*C).  Asserts
      * every differing total is explained by at most three single-count flips;
      * flipped codes (lower bound) <= 1e-4 of all codes N*G*p*C*A*W;
      * every output whose G totals all match the oracle's is within 1e-5
        relative of the oracle's output;
      * with ``xscale`` [N, G] and ``wscale`` [G, p*C]: every other output is
        within the flips' own effect, sum_g |dT| * xs * ws, of the oracle's, plus
        1e-5 of (|output| + sum_g |T| * xs * ws): the FP32 rounding of a sum of
        reads is relative to its terms' magnitudes, not to a result that they
        (and a bias) nearly cancel.
    Returns a dict of the counts for logging.
    """
    got = got.detach().double().cpu().reshape(got.shape[0], -1)
    expected = expected.detach().double().cpu().reshape(expected.shape[0], -1)
    n, o = expected.shape
    differing, flips, unexplained, mask = count_flips(cfg, got_totals, ref_totals)
    codes = mask.numel() * len(input_layout(cfg)) * len(weight_layout(cfg))
    budget = max(1, 1e-4 * codes)
    report = dict(label=label, totals=mask.numel(), differing=differing, flips=flips,
                  codes=codes, budget=budget)
    assert unexplained == 0, f"{label}: {unexplained} totals differ beyond three code flips"
    assert flips <= budget, f"{label}: {flips} flipped codes > budget {budget:.1f} of {codes}"
    flagged = mask.any(1).reshape(n, -1)[:, :o]
    error = (got - expected).abs()
    clean_bad = ~flagged & (error > 1e-5 * expected.abs()) & (got != expected)
    report["flagged_outputs"] = int(flagged.sum())
    report["clean_inexact"] = int((~flagged & (got != expected)).sum())
    assert not clean_bad.any(), (
        f"{label}: {int(clean_bad.sum())} outputs without a flipped total differ by more than "
        f"1e-5 relative (first {clean_bad.nonzero()[:3].tolist()})")
    if xscale is not None and wscale is not None and flagged.any():
        reference = ref_totals.double().cpu()
        delta = (got_totals.double().cpu() - reference).abs()
        delta = delta.reshape(n, delta.shape[1], -1)[:, :, :o]
        xs = xscale.double().cpu()[:, :, None].abs()
        ws = wscale.double().cpu().reshape(wscale.shape[0], -1)[None, :, :o].abs()
        effect = (delta * xs * ws).sum(1)
        magnitude = (reference.abs().reshape(n, reference.shape[1], -1)[:, :, :o] * xs * ws).sum(1)
        allowed = effect * (1 + 1e-5) + 1e-5 * (expected.abs() + magnitude)
        over = flagged & (error > allowed)
        assert not over.any(), (
            f"{label}: {int(over.sum())} flipped outputs move by more than their flips explain")
    return report


def adc_arguments(q, packed, cfg, conductance, begin=0, end=None):
    """Exact ADC arguments y [N, m*Gr, A, W, (end-begin)*C] (FP64) for injected conductances.

    The reference's count argument (memfast/reference.py:54-60, 96-115) in exact arithmetic:
    value = sum_r da*(g - L)*V*Mw*u with its constants L, V and u = fp32(1 / ((H - L)*V)) (Ma
    cancels), without the roundings of its accumulation; then the S-curve
    y = value / (1 + a*|value|) with its FP32 coefficient a = fp32(alpha / max_w).
    ``conductance`` is the FP32 (or FP64) tensor [m, p, W, R, C] (or with a leading plane
    of one) that both sides read.  Read modes whose argument carries per-read noise
    terms (voltage variation, output-mode or slice_pair read noise) are not covered.
    """
    ni = cfg.nonidealities
    if ni.voltage_variation or (ni.read_variation and ni.read_mode != "shared"):
        raise NotImplementedError("adc_arguments covers write, shared read, drift and SAF noise")
    g = conductance.double().cpu()
    if g.dim() == 6:
        assert g.shape[0] == 1
        g = g[0]
    n, m, r = q.shape
    end = packed.shape[1] if end is None else end
    g = g[:, : end - begin] if g.shape[1] > end - begin else g
    # The reference's constants (memfast/reference.py:23-27, 56, 96-101): the low level and
    # read voltage in the current's dtype, 1 / current_unit rounded to FP32 in the ADC.
    low, volt = float(cfg.low_conductance), float(cfg.read_voltage)
    inverse = 1.0 / ((float(cfg.high_conductance) - low) * volt)
    if not precise_currents(cfg):
        f32 = lambda x: torch.tensor(x, dtype=torch.float32).double().item()
        low, volt = f32(low), f32(volt)
    inverse = torch.tensor(inverse, dtype=torch.float32).double().item()
    rows, groups = read_rows(cfg), reads_per_array(cfg)
    width, c = end - begin, cfg.array_size[1]
    out = torch.zeros((n, m * groups, len(input_layout(cfg)), len(weight_layout(cfg)), width * c),
                      dtype=torch.float64)
    for ai, (sa, ma, _) in enumerate(input_layout(cfg)):
        da = ((q.long() >> sa) & ma).double()                       # [n, m, r]
        for wi, (_, mw, _) in enumerate(weight_layout(cfg)):
            effective = (g[:, :, wi] - low) * (volt * mw * inverse)    # [m, t, r, c]
            maximum = adc_maxima(cfg)[wi]
            coeff = torch.tensor(ni.adc_nonlinearity / maximum, dtype=torch.float32).item()
            for j in range(groups):
                lo, hi = j * rows, min((j + 1) * rows, r)
                value = torch.einsum("nir,itrc->nitc", da[:, :, lo:hi], effective[:, :, lo:hi])
                if ni.adc_nonlinearity:
                    value = value / (1 + coeff * value.abs())
                out[:, j::groups, ai, wi] = value.reshape(n, m, width * c)
    return out


def boundary_flips(cfg, got_totals, ref_totals, arguments, tolerance):
    """Explain every differing slice total by rounding-boundary flips.

    ``arguments`` [N, G, A, W, p*C] are the exact ADC arguments (adc_arguments).  A pair
    may flip only where its argument lies within ``tolerance * max(1, |y|)`` of a
    rounding boundary: a half-integer inside [0, max_w], where round() changes value.
    Each differing total must equal a signed sum of at most three such pairs' fa*fw.
    Returns (differing totals, flips, the largest relative boundary distance of a flipped
    pair, list of unexplained (index, difference, nearest relative distances))."""
    diff = (got_totals.double().cpu() - ref_totals.double().cpu())
    n, groups = diff.shape[0], diff.shape[1]
    diff = diff.reshape(n, groups, -1)
    y = arguments
    maxima = torch.tensor(adc_maxima(cfg), dtype=torch.float64)[None, None, None, :, None]
    clamped = y.clamp(min=-0.5 * torch.ones_like(y), max=maxima + 0.5)
    distance = (clamped - clamped.floor() - 0.5).abs()
    # Boundaries only at half-integers in [0.5, max - 0.5] (the clamp is exact elsewhere).
    inside = (y > 0) & (y < maxima)
    near = inside & (distance <= tolerance * y.abs().clamp(min=1.0))
    factors = [[fa * fw for _, _, fw in weight_layout(cfg)] for _, _, fa in input_layout(cfg)]
    relative = distance / y.abs().clamp(min=1.0)
    flips, worst = 0, 0.0
    unexplained = []
    for index in diff.nonzero().tolist():
        v, g_, col = index
        want = int(diff[v, g_, col])
        pairs_near = near[v, g_, :, :, col].nonzero().tolist()
        candidates = [factors[a][w] for a, w in pairs_near]
        found = None
        for count in range(1, 4):
            for chosen in itertools.combinations(range(len(candidates)), count):
                for signs in itertools.product((1, -1), repeat=count):
                    if sum(s * candidates[i] for s, i in zip(signs, chosen)) == want:
                        found = chosen
                        break
                if found:
                    break
            if found:
                break
        if found:
            flips += len(found)
            for i in found:
                a, w = pairs_near[i]
                worst = max(worst, float(relative[v, g_, a, w, col]))
        else:
            unexplained.append((index, want,
                                sorted(relative[v, g_, :, :, col].flatten().tolist())[:3]))
    return int((diff != 0).sum()), flips, worst, unexplained
