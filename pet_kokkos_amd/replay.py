"""A caller's repeated device work kept as recorded torch CUDA (HIP) graphs and
replayed with one call -- the role the reference gives its graph cache
(include/pet/graph.hpp of peterspackman/pet-kokkos) for a Python caller.

``StepRecorder.launch(sig, work)`` runs ``work()`` eagerly for the signature's
first ``warm_runs`` calls (so every lazily grown buffer has its final address),
records it into a graph on the next call and replays it, and from then on only
replays it: the same kernels in the same order on the same buffers, so the
results are bit-identical to an eager run. ``sig`` is any hashable value that
names everything the work depends on (shapes, flags, the tensors it reads and
writes). The work's return value is kept with the graph and returned by every
replay; its tensors hold the replay's results. Live graphs are held in recency
order, the least recently replayed dropped past ``max_live``. A signature whose
recording fails (work that synchronises or allocates outside torch) becomes
eager-only; the others keep recording. ``counters`` reports what happened.

Nothing this library enqueues records a memset node: it clears with kernels
(torch's ``zero_`` is a fill kernel).
"""
from __future__ import annotations

import collections
import dataclasses

import torch


@dataclasses.dataclass
class Counters:
    eager: int = 0      # calls run eagerly (warming or eager-only)
    records: int = 0    # graphs recorded
    launches: int = 0   # graph replays (a record's first included)
    refusals: int = 0   # recordings that failed (signature now eager-only)
    evictions: int = 0  # graphs dropped to stay within max_live


class StepRecorder:
    def __init__(self, warm_runs: int = 1, max_live: int = 8):
        self.warm_runs = max(0, int(warm_runs))
        self.max_live = max(1, int(max_live))
        self.counters = Counters()
        self._warm: dict = {}  # sig -> eager runs so far, or None for eager-only
        self._live: collections.OrderedDict = collections.OrderedDict()  # sig -> (graph, output), oldest first

    @property
    def live(self) -> int:
        return len(self._live)

    def launch(self, sig, work):
        hit = self._live.get(sig)
        if hit is not None:
            self._live.move_to_end(sig)
            return self._replay(*hit)
        if len(self._warm) >= 4 * self.max_live and sig not in self._warm:
            self._warm.clear()  # keep the table bounded for callers cycling through many signatures
        runs = self._warm.setdefault(sig, 0)
        if runs is None or runs < self.warm_runs:
            if runs is not None:
                self._warm[sig] = runs + 1
            self.counters.eager += 1
            return work()
        graph = torch.cuda.CUDAGraph()
        try:
            torch.cuda.synchronize()
            with torch.cuda.graph(graph):
                out = work()
        except RuntimeError:
            torch.cuda.synchronize()
            self._warm[sig] = None
            self.counters.refusals += 1
            self.counters.eager += 1
            return work()  # the failed recording ran nothing
        del self._warm[sig]
        self.counters.records += 1
        self._live[sig] = (graph, out)
        while len(self._live) > self.max_live:
            self._live.popitem(last=False)
            self.counters.evictions += 1
        return self._replay(graph, out)  # recording does not run the work

    def _replay(self, graph, out):
        self.counters.launches += 1
        graph.replay()
        return out

    def forget(self) -> None:
        """Drop every graph and signature (e.g. when the buffers they name change)."""
        self._live.clear()
        self._warm.clear()
