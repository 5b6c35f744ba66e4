"""A reduced PET whose energy is a closed form (tests/test_gpu_model_properties.py
and tests/test_oracle_model.py use it to pin the model's composition).

With every attention output linear, centre expansion, MLP output layer and
combination output layer zeroed (weights and biases), the feedforward
featurizer's layers (reference src/feedforward.cpp:34-336) leave the node
features at their species embedding (each block adds exactly zero to them) and
the edge features follow ie <- ie + compress_L(ie) (the attention block and
the edge MLP add zero, the combination MLP adds zero); the energy is the
readout of those (src/ops.cpp:406-418): per atom, scale (node_head(emb) +
sum over its edges cut * edge_head(ie)) + composition. Computed here in numpy
float64 from positions, so central differences give its forces.
"""
from __future__ import annotations

import numpy as np

from pet_kokkos_amd import systems, weights


def reduced_weights(h, seed):
    w = weights.random_weights(h, seed)
    for k in w:
        if any(s in k for s in (".attention.output_linear.", ".center_expansion.", ".center_mlp.w_out.",
                                ".mlp.w_out.")) or (k.startswith("combination_mlps.") and ".2." in k):
            w[k] = np.zeros_like(w[k])
    return w


def closed_form_energy(h, w, comp, s, energy_scale=1.0):
    """The reduced PET's per-atom energies, numpy float64, from positions."""
    e = systems.neighbor_list(s, h.cutoff)
    sp = np.array([list(h.atomic_types).index(int(z)) for z in s.numbers])
    nsp = sp[e.neigh]
    x = np.asarray(s.positions, np.float64)
    v = x[e.neigh] + e.shift @ s.cell - x[e.centre]
    d = np.sqrt((v * v).sum(1))
    t = np.clip((d - (h.cutoff - h.cutoff_width)) / h.cutoff_width, 0.0, 1.0)
    cut = 0.5 * (1.0 + np.cos(np.pi * t))  # cosine
    x4 = np.concatenate([v, d[:, None]], 1)
    lin = lambda a, k: a @ w[k + ".weight"].T + w[k + ".bias"]
    silu = lambda a: a / (1.0 + np.exp(-a))
    ie = w["edge_embedder.weight"][nsp]
    for L in range(h.num_gnn_layers):
        g = f"gnn_layers.{L}"
        emb = lin(x4, g + ".edge_embedder")
        blocks = [emb, ie] if L == 0 else [emb, w[g + ".neighbor_embedder.weight"][nsp], ie]
        ie = ie + lin(silu(lin(np.concatenate(blocks, 1), g + ".compress.0")), g + ".compress.2")

    def head(a, side):
        y = silu(lin(silu(lin(a, f"{side}_heads.energy.0.0")), f"{side}_heads.energy.0.2"))
        return lin(y, f"{side}_last_layers.energy.0.energy___0")[:, 0]

    net = head(w["node_embedders.0.weight"][sp], "node")
    np.add.at(net, e.centre, cut * head(ie, "edge"))
    return energy_scale * net + np.asarray(comp)[sp]


