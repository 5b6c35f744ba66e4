"""Random-init PET weights in the reference checkpoint's names and layouts.

The reference reads a metatrain PET checkpoint converted to safetensors plus a
JSON of hyperparameters (peterspackman/pet-kokkos src/checkpoint.cpp:12-52,
include/pet/config.hpp:30-70) and loads the tensors named in
src/model.cpp:180-289. There is no network here for a published checkpoint, so
the benchmark models are random-init with exactly those names and shapes
(torch Linear layout [out, in]; a SwiGLU ``w_in`` as metatrain stores it, the
value rows [0, F) then the gate rows [F, 2F); ``compress.0`` unfolded, its
input columns [edge_emb | neighbour/edge embedding | input_edge]).

Both featurizers the reference implements (src/model.cpp:326-340): the
feedforward one (PreLN, RMSNorm, SwiGLU, d_node != d_pet) and the residual one
(PostLN, LayerNorm, SiLU, d_node == d_pet, a readout after every GNN layer).
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass(frozen=True)
class Hypers:
    """The subset of metatrain's PET hyperparameters evaluation needs
    (include/pet/config.hpp:30-70)."""
    d_pet: int = 128
    d_node: int = 256
    d_head: int = 128
    d_feedforward: int = 512
    num_heads: int = 4
    num_gnn_layers: int = 2
    num_attention_layers: int = 2
    cutoff: float = 4.5
    cutoff_width: float = 0.5
    cutoff_function: str = "cosine"  # bump | cosine | smooth
    attention_temperature: float = 1.0
    atomic_types: tuple = (1, 6, 8)
    featurizer: str = "feedforward"  # or "residual"

    @property
    def residual(self) -> bool:
        return self.featurizer == "residual"

    @property
    def head_dim(self) -> int:
        return self.d_pet // self.num_heads

    @property
    def n_species(self) -> int:
        return len(self.atomic_types)

    @property
    def center_width(self) -> int:
        """center_mlp.w_in's rows: SwiGLU over 2 d_node (tools/roofline.py:113)."""
        return 4 * self.d_node

    @property
    def edge_width(self) -> int:
        """mlp.w_in's rows: SwiGLU over d_feedforward (tools/roofline.py:112),
        d_feedforward for the residual featurizer's SiLU MLP."""
        return self.d_feedforward if self.residual else 2 * self.d_feedforward


# The E+F workloads: configs[1] (water-648) and configs[4] (batch of 32). The
# PET shape of configs[1] is given (d 128, 4 heads, 2 x 2 layers, FFN 512);
# d_node and d_head, which the feedforward featurizer needs and the config does
# not name, are 2 d_pet and 128. configs[4] gives d 512, 8 heads (head_dim 64),
# 2 x 2 layers; its FFN width is metatrain's default 2 d_pet.
MODELS = {
    "c2": Hypers(d_pet=128, d_node=256, d_head=128, d_feedforward=512, num_heads=4),
    "c5": Hypers(d_pet=512, d_node=1024, d_head=128, d_feedforward=1024, num_heads=8),
    # small models for the tests
    "tiny": Hypers(d_pet=64, d_node=128, d_head=32, d_feedforward=128, num_heads=4),
    "tiny-residual": Hypers(d_pet=64, d_node=64, d_head=32, d_feedforward=128, num_heads=4,
                            featurizer="residual"),
    # widths whose quarter does not divide 256 and a head_dim of 16: the
    # library's scalar fallbacks of its row passes, and masked norm lanes
    "odd": Hypers(d_pet=48, d_node=72, d_head=40, d_feedforward=36, num_heads=3),
    "odd-residual": Hypers(d_pet=48, d_node=48, d_head=40, d_feedforward=36, num_heads=3,
                           featurizer="residual"),
    # head_dims the LDS-staged attention kernels do not hold (the streaming
    # kernels): 20 (a multiple of 4) and 10 (not even that; widths of 30)
    "hd20": Hypers(d_pet=60, d_node=120, d_head=40, d_feedforward=48, num_heads=3),
    "hd10-residual": Hypers(d_pet=30, d_node=30, d_head=20, d_feedforward=24, num_heads=3, featurizer="residual"),
    # the residual family at configs[1]'s shape
    "c2-residual": Hypers(d_pet=128, d_node=128, d_head=128, d_feedforward=512, num_heads=4,
                          featurizer="residual"),
}


def random_weights(h: Hypers, seed: int = 0) -> dict[str, np.ndarray]:
    """Every tensor the reference loads for this family (src/model.cpp:226-288),
    float64: linear weights N(0, 1/fan_in), biases N(0, 0.1^2), norm weights
    1 + N(0, 0.1^2), embeddings N(0, 1)."""
    rng = np.random.default_rng(seed)
    w: dict[str, np.ndarray] = {}
    D, Dn, Dh, ns = h.d_pet, h.d_node, h.d_head, h.n_species

    def lin(name, out, inp):
        w[name + ".weight"] = rng.standard_normal((out, inp)) / np.sqrt(inp)
        w[name + ".bias"] = 0.1 * rng.standard_normal(out)

    def norm(name, width, bias=False):
        w[name + ".weight"] = 1.0 + 0.1 * rng.standard_normal(width)
        if bias:
            w[name + ".bias"] = 0.1 * rng.standard_normal(width)

    w["edge_embedder.weight"] = rng.standard_normal((ns, D))
    R = h.num_gnn_layers if h.residual else 1  # readouts
    for i in range(R):
        w[f"node_embedders.{i}.weight"] = rng.standard_normal((ns, Dn))
    for L in range(h.num_gnn_layers):
        g = f"gnn_layers.{L}"
        lin(g + ".edge_embedder", D, 4)
        if L > 0:
            w[g + ".neighbor_embedder.weight"] = rng.standard_normal((ns, D))
        lin(g + ".compress.0", D, (2 if L == 0 else 3) * D)
        lin(g + ".compress.2", D, D)
        for a in range(h.num_attention_layers):
            t = f"{g}.trans.layers.{a}"
            lin(t + ".attention.input_linear", 3 * D, D)
            lin(t + ".attention.output_linear", D, D)
            norm(t + ".norm_attention", D, bias=h.residual)
            norm(t + ".norm_mlp", D, bias=h.residual)
            lin(t + ".mlp.w_in", h.edge_width, D)
            lin(t + ".mlp.w_out", D, h.d_feedforward)
            if h.residual:
                continue
            lin(t + ".center_contraction", D, Dn)
            lin(t + ".center_expansion", Dn, D)
            norm(t + ".norm_center_features", Dn)
            lin(t + ".center_mlp.w_in", h.center_width, Dn)
            lin(t + ".center_mlp.w_out", Dn, h.center_width // 2)
        if h.residual:
            continue
        norm(f"combination_norms.{L}", 2 * D, bias=True)
        lin(f"combination_mlps.{L}.0", 2 * D, 2 * D)
        lin(f"combination_mlps.{L}.2", D, 2 * D)
    for i in range(R):
        lin(f"node_heads.energy.{i}.0", Dh, Dn)
        lin(f"node_heads.energy.{i}.2", Dh, Dh)
        lin(f"edge_heads.energy.{i}.0", Dh, D)
        lin(f"edge_heads.energy.{i}.2", Dh, Dh)
        lin(f"node_last_layers.energy.{i}.energy___0", 1, Dh)
        lin(f"edge_last_layers.energy.{i}.energy___0", 1, Dh)
    return w


def random_composition(h: Hypers, seed: int = 0) -> np.ndarray:
    """Per-species energy offsets (the checkpoint's composition model)."""
    return np.random.default_rng(seed + 7).standard_normal(h.n_species)
