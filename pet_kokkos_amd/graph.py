"""Record-and-replay of the path's device work as one HIP graph launch, the
role of the reference's GraphCache (include/pet/graph.hpp) for a caller in
Python.

For a small structure an evaluation is a few dozen short kernels whose launch
cost is most of its time. ``GraphCache.run(key, work)`` runs ``work`` eagerly
the first time it sees ``key``, captures it into a graph the second time (the
work's allocations then come from the graph's private pool and are reused), and
replays the graph from then on: the same kernels, in the same order, on the same
buffers, so the results are bit-identical to an eager run. The key must name
everything the recorded work depends on (shapes and the tensors it reads and
writes), since a replay reuses the recorded pointers. The least recently used
graph is dropped past ``keep``. A capture that fails switches the cache to
eager work for good.

Nothing in the captured path records a memset node: the library clears with
kernels (and torch's ``zero_`` is a fill kernel).
"""
from __future__ import annotations

import torch


class GraphCache:
    def __init__(self, keep: int = 8):
        self.keep = keep
        self._graphs: dict = {}  # key -> [graph, output, last use]
        self._seen: list = []
        self._tick = 0
        self.broken = False

    def run(self, key, work):
        """work() -> output; the output of a replayed graph is the recorded one
        (its tensors hold the replay's results)."""
        if self.broken:
            return work()
        self._tick += 1
        hit = self._graphs.get(key)
        if hit is not None:
            hit[2] = self._tick
            hit[0].replay()
            return hit[1]
        if key not in self._seen:
            self._seen.append(key)
            if len(self._seen) > 2 * self.keep:
                self._seen.pop(0)
            return work()  # first sight: eagerly
        g = torch.cuda.CUDAGraph()
        try:
            torch.cuda.synchronize()
            with torch.cuda.graph(g):
                out = work()
        except RuntimeError:
            self.broken = True
            torch.cuda.synchronize()
            return work()
        if len(self._graphs) >= self.keep:
            lru = min(self._graphs, key=lambda k: self._graphs[k][2])
            del self._graphs[lru]
        self._graphs[key] = [g, out, self._tick]
        g.replay()  # the capture recorded the work without running it
        return out

    def clear(self) -> None:
        self._graphs.clear()
        self._seen.clear()
