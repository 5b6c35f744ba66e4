"""The path recorded as HIP graphs and replayed (pet_kokkos_amd.replay, the
role of the reference's graph cache, include/pet/graph.hpp): every replay gives
the eager run's bits, with the program's own eager work and synchronisations
between the replays; the core kernels, the op level with rocBLAS's GEMMs, the
layer level with the token norm, and the forces' edge term and fold."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from pet_kokkos_amd import attention as A
from pet_kokkos_amd import forces as F
from pet_kokkos_amd import replay as G
from pet_kokkos_amd import layer as L
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu


def _setup(device):
    cfg = systems.CONFIGS["c1"]
    s = systems.build_structure(cfg.structure, 0)
    e = systems.neighbor_list(s, cfg.cutoff)
    N = len(s.positions)
    tk = systems.tokens_from_edges(N, e, cfg.cutoff, cfg.width)
    pk = F.PackedEdges.from_host(systems.packed_edges(N, e, cfg.cutoff, cfg.width), device)
    H, hd, D = cfg.heads, cfg.head_dim, cfg.d_model
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    r = lambda *shape: torch.randn(shape, device=device, generator=gen)
    t = dict(tok=r(tk.n_rows, D), nw=1 + 0.1 * r(D), w_in=r(3 * D, D) / D ** 0.5, b_in=0.1 * r(3 * D),
             w_out=r(D, D) / D ** 0.5, b_out=0.1 * r(D), out_adj=r(tk.n_rows, D), x4=r(pk.n_edges, 4))
    t["qkv"] = torch.addmm(t["b_in"], t["tok"], t["w_in"].t()).contiguous()
    t["off"] = torch.from_numpy(tk.off).to(device)
    t["cf"] = torch.from_numpy(tk.cf_seq).to(device)
    return cfg, tk, pk, t


def test_graph_replays_are_bit_identical(device):
    print("[gpu] graph replay c1: core, op level, layer level, forces", flush=True)
    cfg, tk, pk, t = _setup(device)
    H, hd, D, N, S, T = cfg.heads, cfg.head_dim, cfg.d_model, tk.n_atoms, tk.slots, tk.n_rows
    tks = A.Tokens(t["off"], N)
    ws = A.Workspace(device)
    out = torch.empty((T, D), device=device)
    in_adj = torch.empty((T, D), device=device)
    tadj = torch.empty((T, D), device=device)
    csa = torch.empty((N, S), device=device)
    merged = torch.empty((T, D), device=device)
    ml = torch.empty((N * H * S, 2), device=device)
    qa = torch.empty((T, 3 * D), device=device)
    cfh = torch.empty((N, H, S), device=device)
    soff = torch.tensor([0, N], dtype=torch.int32, device=device)

    def work():
        csa.zero_()  # the accumulated outputs start from zero (fill kernels)
        tadj.zero_()
        A.attn_fwd(t["qkv"], t["off"], t["cf"], H, hd, merged=merged, ml=ml)
        A.attn_bwd(t["qkv"], t["off"], t["out_adj"], merged, ml, t["cf"], H, hd, cf_seq_adj=csa, qkv_adj=qa, cfh=cfh)
        A.attention(ws, "op", out, t["qkv"], t["cf"], t["w_out"], t["b_out"], tks, S, H, hd, 1.0, True)
        A.attention_bwd(ws, "op", in_adj, csa, t["out_adj"], t["qkv"], t["cf"], t["w_in"], t["w_out"], tks, S, H,
                        hd, 1.0, 0.0)
        L.attention_layer(ws, "ly", out, t["tok"], t["nw"], None, t["w_in"], t["b_in"], t["cf"], t["w_out"],
                          t["b_out"], tks, S, H, hd, 1.0)
        L.attention_layer_bwd(ws, "ly", tadj, csa, t["out_adj"], t["tok"], t["nw"], None, t["w_in"], t["b_in"],
                              t["cf"], t["w_out"], tks, S, H, hd, 1.0)
        return F.forces_and_virial(pk, N, soff, t["x4"], None, csa, cfg.width, "cosine", -1.0)

    def snapshot(res):
        torch.cuda.synchronize()
        return [x.clone() for x in (merged, ml, qa, cfh, out, in_adj, tadj, csa, *res)]

    eager = snapshot(work())
    cache = G.StepRecorder()
    key = ("c1", T, D)
    first = snapshot(cache.launch(key, work))  # warming: eager
    for a, b in zip(eager, first):
        assert torch.equal(a, b)
    for rep in range(4):
        res = cache.launch(key, work)  # recorded on the second call, replayed after
        got = snapshot(res)
        assert cache.counters.refusals == 0
        for a, b in zip(eager, got):
            assert torch.equal(a, b), f"replay {rep} differs"
        # the program's own eager work between replays
        scratch = torch.randn((T, D), device=device)
        L.norm_rows(scratch, scratch, t["nw"], None)
        torch.cuda.synchronize()
    n = cache.counters
    assert cache.live == 1 and n.records == 1 and n.eager == 1 and n.launches == 4, n


def test_recorder_bounds(device):
    # past max_live the least recently replayed graph is dropped
    x = torch.zeros(1024, device=device)
    cache = G.StepRecorder(warm_runs=0, max_live=2)
    for k in (1, 2, 1, 3, 1):
        out = cache.launch(("add", k), lambda k=k: x.add(k))
        torch.cuda.synchronize()
        assert torch.all(out == k)
    n = cache.counters
    assert n.records == 3 and n.evictions == 1 and cache.live == 2 and n.launches == 5, n
