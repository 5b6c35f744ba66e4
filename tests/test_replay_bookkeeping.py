"""The step recorder's bookkeeping (pet_kokkos_amd.replay.StepRecorder) on the
CPU, with torch's graph calls replaced by stand-ins: warm runs, recording,
replays, recency eviction, and a refused recording that leaves only its own
signature eager. (A refused capture cannot be provoked on a GPU without
invalidating the process's capture state, so this part is tested here.)"""
from __future__ import annotations

import contextlib

import pytest
import torch

from pet_kokkos_amd import replay


class FakeGraph:
    replays = 0

    def replay(self):
        FakeGraph.replays += 1


@pytest.fixture
def fake_cuda(monkeypatch):
    state = {"refuse": False}

    @contextlib.contextmanager
    def graph(g):
        if state["refuse"]:
            raise RuntimeError("operation not permitted when stream is capturing")
        yield

    monkeypatch.setattr(torch.cuda, "CUDAGraph", FakeGraph)
    monkeypatch.setattr(torch.cuda, "graph", graph)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    FakeGraph.replays = 0
    return state


def test_warm_record_replay(fake_cuda):
    r = replay.StepRecorder(warm_runs=2, max_live=4)
    calls = []
    for _ in range(5):
        r.launch("a", lambda: calls.append(1) or "out")
    n = r.counters
    # two eager runs, one recording (which runs nothing), then replays
    assert len(calls) == 3 and n.eager == 2 and n.records == 1 and n.launches == 3
    assert FakeGraph.replays == 3 and r.live == 1


def test_eviction_by_recency(fake_cuda):
    r = replay.StepRecorder(warm_runs=0, max_live=2)
    for k in ("a", "b", "a", "c", "b"):
        r.launch(k, lambda: k)
    n = r.counters
    # a, b recorded; a replayed; c recorded and b (least recent) dropped; b recorded again
    assert n.records == 4 and n.evictions == 2 and n.launches == 5 and r.live == 2


def test_refusal_is_per_signature(fake_cuda):
    r = replay.StepRecorder(warm_runs=1, max_live=4)
    r.launch("good", lambda: 0)
    r.launch("good", lambda: 0)
    fake_cuda["refuse"] = True
    ran = []
    for _ in range(3):
        r.launch("bad", lambda: ran.append(1))
    fake_cuda["refuse"] = False
    r.launch("good", lambda: 0)
    r.launch("bad", lambda: ran.append(1))
    n = r.counters
    assert n.refusals == 1 and len(ran) == 4  # every "bad" call ran eagerly, once refused always eager
    assert n.records == 1 and n.launches == 2 and r.live == 1


def test_forget(fake_cuda):
    r = replay.StepRecorder(warm_runs=0)
    r.launch("a", lambda: 0)
    r.forget()
    assert r.live == 0
    r.launch("a", lambda: 0)
    assert r.counters.records == 2
