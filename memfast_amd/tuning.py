"""Tuned mode: a per-shape search over the read kernels' own launch parameters.

The reference's tuned mode (memfast/simulator.py:27-45, :195-347) traverses a
grid of CUDA launch shapes (arrays x vectors x columns x workers), keeps every
candidate whose output is bit-identical to the default schedule's, times each
once and caches the fastest per (configuration, hardware, shape, dtype,
sources, workspace budget, grid) in a JSON file.  The same protocol runs here
over the parameters the gfx950 kernels actually have, chosen by the kernel
``mf_mm_kernel`` selects for the shape:

* ideal-device MFMA read (kernel 1): the block tile, 64 or 128 vectors by 64
  columns (the taller tile only with 32-row reads);
* noisy-device MFMA read (kernel 2): how many chunks a block's reads are split
  into (0 automatic, 1 never, 2, 4, 8); a split writes integer totals to the
  workspace, so its scratch counts against the budget;
* wide noisy-device MFMA read (kernel 3): the LDS capacity per read (0
  automatic, 24, 36 or 72 conductance fragments), which sets blocks per CU;
* general kernel (kernel 0): one tiling, so one candidate.

A schedule keeps the reference's keys (arrays, vectors, columns, workers) for
reports and adds ``tile``, ``split`` and ``tier``; ``schedule_variant`` turns
it into the ``variant`` word of mf_mm.  Results never depend on the schedule,
which is what the bit-exact candidate check enforces.
"""

import hashlib
import json
import time
from dataclasses import asdict

import torch

from . import hip

TILES = {"64x64": 2, "128x64": 1}     # mf_mm variant tile field of each block tile
SPLITS = (1, 2, 4, 8)                 # explicit read splits of the noisy read
TIERS = {1: 24, 2: 36, 3: 72}         # LDS fragments per read of each wide tier
DEFAULT_VARIANT = TILES["64x64"]      # schedule_variant(default_schedule(config))


def default_schedule(config):
    """The schedule default mode runs (keys of memfast/simulator.py:27-28 plus the kernels')."""
    return dict(arrays=2, vectors=2, columns=4, workers=min(2, len(config.weight_layout)),
                tile="64x64", split=0, tier=0)


def schedule_variant(schedule):
    """mf_mm's ``variant`` word for a schedule (missing keys take their defaults)."""
    return hip.variant_word(TILES[schedule.get("tile", "64x64")], schedule.get("split", 0),
                            schedule.get("tier", 0))


def read_kernel(config, n, arrays, partitions):
    """The read kernel (0-3) ``hip.mm`` launches for n vectors through m x p arrays."""
    return hip.mm_kernel(config, n, arrays, partitions)


def schedule_grid(config, n, partitions, arrays=None):
    """Candidate schedules for n input vectors through ``arrays`` x ``partitions`` arrays.

    Without ``arrays`` (the reference's signature) the kernel is unknown and only
    the default schedule is declared."""
    base = default_schedule(config)
    kernel = None if arrays is None else read_kernel(config, n, arrays, partitions)
    if kernel == 1:
        tiles = ["64x64"] + (["128x64"] if config.read_rows == 32 else [])
        return [dict(base, tile=tile) for tile in tiles]
    if kernel == 2:
        reads = arrays * config.reads_per_array
        return [base] + [dict(base, split=split) for split in SPLITS if split <= reads]
    if kernel == 3:
        return [base] + [dict(base, tier=tier) for tier in TIERS]
    return [base]


def workspace_need(config, n, arrays, partitions, schedule):
    """Device bytes a read under ``schedule`` allocates besides its inputs and output: the MFMA
    kernels' scratch (mf_mm_workspace for the schedule's variant) or, for the general kernel
    with device noise, the restored conductance tensor."""
    kernel = read_kernel(config, n, arrays, partitions)
    if kernel:
        return hip.mm_workspace_bytes(config, n, arrays, partitions, schedule_variant(schedule))
    if not hip.needs_conductances(config):
        return 0
    rows, cols = config.array_size
    element = 8 if config.precise_currents else 4
    return (element * hip.restore_planes(config) * arrays * partitions
            * len(config.weight_layout) * rows * cols)


class ScheduleSearch:
    """One tuned selection for a programmed matrix and an input shape.

    ``run`` executes the reference protocol: the first admissible schedule of
    [default, *grid] gives the reference output; a cached winner is accepted only
    after it reproduces that output bit for bit; otherwise every candidate is
    admitted, checked bit for bit, timed, and the fastest is written to the
    cache atomically."""

    TIMED_SAMPLES = 2

    def __init__(self, simulator, matrix, x, q, xscale, event):
        self.simulator, self.matrix = simulator, matrix
        self.x, self.q, self.xscale, self.event = x, q, xscale, event
        self.started = time.perf_counter()
        n, arrays = q.shape[0], q.shape[1]
        self.grid = schedule_grid(simulator.config, n, matrix.p, arrays)
        self.key, self.payload = simulator._key(matrix, x, self.grid)
        self.path = simulator.cache_dir / f"{self.key}.json"
        self.record = dict(key=self.key, layer=matrix.name, shape=list(x.shape),
                           kernel=read_kernel(simulator.config, n, arrays, matrix.p),
                           cache_hit=False, candidates=[], selected=None, complete=False)

    # -- helpers --------------------------------------------------------------
    def _read(self, schedule):
        return self.matrix._execute(self.q, self.xscale, schedule, self.event)

    @staticmethod
    def _same_bits(a, b):
        view = torch.int32 if a.dtype == torch.float32 else torch.int64
        return a.shape == b.shape and torch.equal(a.view(view), b.view(view))

    def _admitted_read(self, schedule):
        """(output, resources), or None when the schedule is infeasible here."""
        try:
            resources = self.simulator._admit(self.matrix, self.q, schedule)
            return self._read(schedule), resources
        except (hip.ResourceError, torch.cuda.OutOfMemoryError):
            torch.cuda.empty_cache()
            return None

    # -- steps ------------------------------------------------------------------
    def _reference_output(self):
        for schedule in [default_schedule(self.simulator.config), *self.grid]:
            admitted = self._admitted_read(schedule)
            if admitted is not None:
                output = admitted[0]
                if not torch.isfinite(output).all():
                    raise FloatingPointError("nonfinite default output during tuning")
                return output
        raise RuntimeError("no feasible reference schedule in the declared grid")

    def _stored_winner(self):
        """The cached winner for this key if the file is readable, complete, written for the
        same fingerprint and names a schedule of the current grid; else None."""
        remembered = self.simulator._selections.get(self.key)
        if remembered is not None:
            return remembered
        if not self.path.is_file():
            return None
        try:
            content = json.loads(self.path.read_text(encoding="utf-8"))
            winner = content["selected"]
            valid = (content["fingerprint"] == self.payload and content["complete"] is True
                     and winner in self.grid)
        except (OSError, KeyError, ValueError, TypeError):
            return None
        return winner if valid else None

    def _time(self, schedule):
        best = None
        for _ in range(self.TIMED_SAMPLES):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            self._read(schedule)
            end.record()
            end.synchronize()
            seconds = start.elapsed_time(end) / 1000
            best = seconds if best is None else min(best, seconds)
        return best

    def _traverse(self, reference):
        for schedule in self.grid:
            candidate = dict(schedule=schedule, status="rejected", timed_samples=0)
            self.record["candidates"].append(candidate)
            try:
                candidate["resources"] = self.simulator._admit(self.matrix, self.q, schedule)
                output = self._read(schedule)
                if not self._same_bits(reference, output):
                    raise RuntimeError("schedule changes output")
                del output
                candidate.update(status="accepted", seconds=self._time(schedule),
                                 timed_samples=self.TIMED_SAMPLES)
            except hip.ResourceError as error:
                candidate["reason"] = str(error)
            except torch.cuda.OutOfMemoryError:
                candidate["reason"] = "HIP out of memory"
                torch.cuda.empty_cache()
        timed = [c for c in self.record["candidates"] if c["status"] == "accepted"]
        if not timed:
            raise RuntimeError("no feasible schedule in the declared grid")
        return min(timed, key=lambda c: c["seconds"])["schedule"]

    def _save(self, winner):
        body = dict(fingerprint=self.payload, complete=True, selected=winner,
                    candidates=self.record["candidates"])
        hip.atomic_write(self.path, json.dumps(body, sort_keys=True).encode())

    def run(self):
        self.simulator.records.append(self.record)
        reference = self._reference_output()
        winner = self._stored_winner()
        if winner is not None:
            admitted = self._admitted_read(winner)
            if admitted is not None:
                if not self._same_bits(reference, admitted[0]):
                    raise RuntimeError("cached schedule changes output")
                self._finish(winner, cache_hit=True)
                return winner
        winner = self._traverse(reference)
        self._save(winner)
        self._finish(winner, cache_hit=False, domain_count=len(self.grid))
        return winner

    def _finish(self, winner, **fields):
        self.record.update(selected=winner, complete=True,
                           preparation_seconds=time.perf_counter() - self.started, **fields)
        self.simulator._selections[self.key] = winner


def selection_key(simulator, matrix, x, grid, fingerprint):
    """(sha256 hex digest, payload) identifying a selection (memfast/simulator.py:195-214):
    configuration, hardware identity, input shape and dtype, output width, sources
    fingerprint, workspace budget and the candidate grid."""
    payload = dict(
        config=asdict(simulator.config),
        hardware=hip.identity(simulator.device),
        shape=list(x.shape),
        output=matrix.out_features,
        dtype=str(x.dtype),
        sources=fingerprint,
        workspace_bytes=simulator.workspace_bytes,
        grid=grid,
    )
    payload = json.loads(json.dumps(payload))
    return hashlib.sha256(json.dumps(payload, sort_keys=True).encode()).hexdigest(), payload
