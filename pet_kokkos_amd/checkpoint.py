"""The reference's converted checkpoint, for either featurizer: <model>.json (hyperparameters, the
species map, composition energies, energy scale) and <model>.safetensors (the
weights under metatrain's names), as peterspackman/pet-kokkos's
tools/convert_pet.py:341-420 writes them and src/checkpoint.cpp:12-141 reads
them.

Reading takes safetensors' own loader (no pickle) and refuses, by name, what
the GPU model does not implement, as the reference's loader does
(src/checkpoint.cpp:136-139, src/model.cpp:326-340): it would otherwise load
and return wrong energies.
"""
from __future__ import annotations

import dataclasses
import json

import numpy as np

from .weights import Hypers

CUTOFF_NAMES = {"Bump": "bump", "Cosine": "cosine"}


@dataclasses.dataclass
class Checkpoint:
    hypers: Hypers
    weights: dict
    energy_scale: float
    composition: np.ndarray  # [n_species] eV
    species_to_index: list  # [Z] -> species index, -1 unsupported


def _refuse(what: str):
    raise ValueError(f"checkpoint: {what} is not implemented by this build")


def load(json_path: str, safetensors_path: str) -> Checkpoint:
    from safetensors.numpy import load_file
    with open(json_path) as f:
        j = json.load(f)
    h = j["hypers"]
    feat = h.get("featurizer_type")
    if feat == "feedforward":
        if h.get("normalization") != "RMSNorm" or h.get("activation") != "SwiGLU" or \
                h.get("transformer_type") != "PreLN":
            _refuse("a feedforward featurizer other than PreLN + RMSNorm + SwiGLU")
        if int(h["d_node"]) == int(h["d_pet"]):
            _refuse("the feedforward featurizer without an expanded central token (d_node == d_pet)")
    elif feat == "residual":
        if h.get("normalization") != "LayerNorm" or h.get("activation") != "SiLU" or \
                h.get("transformer_type") != "PostLN":
            _refuse("a residual featurizer other than PostLN + LayerNorm + SiLU")
        if int(h["d_node"]) != int(h["d_pet"]):
            _refuse("the residual featurizer with an expanded central token (d_node != d_pet)")
    else:
        _refuse(f"featurizer_type {feat!r}")
    if h.get("num_neighbors_adaptive") is not None:
        _refuse("the adaptive cutoff")
    for flag in ("zbl", "long_range_enabled", "system_conditioning"):
        if h.get(flag, False):
            _refuse(flag)
    if "non_conservative" in j or "uncertainty" in j:
        pass  # extra heads; the energy path ignores them
    if h.get("cutoff_function") not in CUTOFF_NAMES:
        _refuse(f"cutoff_function {h.get('cutoff_function')!r}")
    readouts = int(h["num_gnn_layers"]) if feat == "residual" else 1
    if int(h.get("num_readout_layers", readouts)) != readouts:
        _refuse(f"num_readout_layers != {readouts} for the {feat} featurizer")
    s2i = [int(x) for x in j["species_to_index"]]
    n_species = int(j["n_species"])
    types = [0] * n_species
    for z, i in enumerate(s2i):
        if i >= 0:
            types[i] = z
    hy = Hypers(d_pet=int(h["d_pet"]), d_node=int(h["d_node"]), d_head=int(h["d_head"]),
                d_feedforward=int(h["d_feedforward"]), num_heads=int(h["num_heads"]),
                num_gnn_layers=int(h["num_gnn_layers"]), num_attention_layers=int(h["num_attention_layers"]),
                cutoff=float(h["cutoff"]), cutoff_width=float(h["cutoff_width"]),
                cutoff_function=CUTOFF_NAMES[h["cutoff_function"]],
                attention_temperature=float(h.get("attention_temperature", 1.0)), atomic_types=tuple(types),
                featurizer=feat)
    if int(h.get("head_dim", hy.head_dim)) != hy.head_dim:
        raise ValueError("checkpoint: head_dim != d_pet / num_heads")
    w = {k: np.asarray(v, dtype=np.float64) for k, v in load_file(safetensors_path).items()}
    return Checkpoint(hy, w, float(j["energy_scale"]), np.asarray(j["composition_energies"], dtype=np.float64), s2i)


def save(prefix: str, h: Hypers, weights: dict, composition, energy_scale: float = 1.0) -> tuple[str, str]:
    """Write <prefix>.json and <prefix>.safetensors in the converter's format
    (float32 tensors, as tools/convert_pet.py:405-420 stores them)."""
    from safetensors.numpy import save_file
    zmax = max(h.atomic_types)
    s2i = [-1] * (zmax + 1)
    for i, z in enumerate(h.atomic_types):
        s2i[z] = i
    inv = {v: k for k, v in CUTOFF_NAMES.items()}
    meta = {
        "format_version": 1, "architecture": "pet", "target": "energy",
        "hypers": {"d_pet": h.d_pet, "d_head": h.d_head, "d_node": h.d_node, "d_feedforward": h.d_feedforward,
                   "num_heads": h.num_heads, "head_dim": h.head_dim,
                   "num_attention_layers": h.num_attention_layers, "num_gnn_layers": h.num_gnn_layers,
                   "num_readout_layers": h.num_gnn_layers if h.residual else 1,
                   "normalization": "LayerNorm" if h.residual else "RMSNorm",
                   "activation": "SiLU" if h.residual else "SwiGLU",
                   "transformer_type": "PostLN" if h.residual else "PreLN", "featurizer_type": h.featurizer,
                   "attention_temperature": h.attention_temperature, "cutoff": h.cutoff,
                   "cutoff_width": h.cutoff_width, "cutoff_function": inv[h.cutoff_function],
                   "num_neighbors_adaptive": None, "adaptive_cutoff_method": "grid",
                   "cutoff_width_adaptive": h.cutoff_width, "system_conditioning": False, "max_charge": 10,
                   "max_spin_multiplicity": 10, "zbl": False, "long_range_enabled": False},
        "length_unit": "angstrom", "energy_unit": "eV", "energy_scale": float(energy_scale),
        "n_species": h.n_species, "atomic_types": list(h.atomic_types), "species_to_index": s2i,
        "composition_energies": [float(c) for c in composition],
    }
    jp, sp = prefix + ".json", prefix + ".safetensors"
    with open(jp, "w") as f:
        json.dump(meta, f, indent=2)
    save_file({k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}, sp)
    return jp, sp
