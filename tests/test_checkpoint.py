"""The converted-checkpoint format (<model>.json + <model>.safetensors, the
reference's tools/convert_pet.py and src/checkpoint.cpp): a round trip, and
the models the GPU path does not implement refused by name."""
from __future__ import annotations

import json

import numpy as np
import pytest

from pet_kokkos_amd import checkpoint, weights


@pytest.mark.parametrize("name", ["tiny", "tiny-residual"])
def test_round_trip(tmp_path, name):
    h = weights.MODELS[name]
    w = weights.random_weights(h, 3)
    comp = weights.random_composition(h)
    jp, sp = checkpoint.save(str(tmp_path / "m"), h, w, comp, energy_scale=1.5)
    c = checkpoint.load(jp, sp)
    assert c.hypers == h
    assert c.energy_scale == 1.5
    assert np.array_equal(c.composition, comp)
    assert c.species_to_index[1] == 0 and c.species_to_index[6] == 1 and c.species_to_index[8] == 2
    assert c.species_to_index[7] == -1
    assert set(c.weights) == set(w)
    for k, v in w.items():
        assert c.weights[k].shape == v.shape
        assert np.array_equal(c.weights[k], v.astype(np.float32).astype(np.float64)), k


@pytest.mark.parametrize("edit", [
    lambda h: h.update(featurizer_type="residual"),  # with RMSNorm / SwiGLU / PreLN and d_node != d_pet
    lambda h: h.update(featurizer_type="other"),
    lambda h: h.update(normalization="LayerNorm"),
    lambda h: h.update(num_neighbors_adaptive=30.0),
    lambda h: h.update(zbl=True),
    lambda h: h.update(long_range_enabled=True),
    lambda h: h.update(d_node=h["d_pet"]),
])
def test_refuses_unimplemented(tmp_path, edit):
    h = weights.MODELS["tiny"]
    jp, sp = checkpoint.save(str(tmp_path / "m"), h, weights.random_weights(h, 0), weights.random_composition(h))
    meta = json.load(open(jp))
    edit(meta["hypers"])
    json.dump(meta, open(jp, "w"))
    with pytest.raises(ValueError, match="not implemented"):
        checkpoint.load(jp, sp)
