"""Pins of the whole-model oracle (oracle/pet_model.py), run without a GPU.

The reference's golden files need published weights that are absent, and
PET is not rotation-invariant by construction (it reads raw Cartesian edge
vectors), so the oracle is pinned by:

  attention      against the C oracle (itself pinned by brute force, torch
                 SDPA and finite differences in tests/test_oracle.py);
  norms          against torch's rms_norm / layer_norm;
  edge grads     central differences of the energy in each edge vector;
  permutation    relabelling atoms permutes per-atom energies and forces;
  extensivity    a periodic supercell's per-atom energies equal the cell's;
  translation    moving every atom leaves energy and forces unchanged;
  fold           forces from the edge gradients against central differences
                 of the energy in atom positions;
  fp32 / fp64    the two precisions agree to fp32 rounding;
for both featurizers (feedforward and residual).

The order in which the layers are composed has no independent vector here:
beyond these checks the model's parity with the reference is unpinned.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import pet_model as om
from pet_kokkos_amd import systems, weights
from pet_kokkos_amd.model import species_index

H = weights.MODELS["tiny"]
FAMILIES = ["tiny", "tiny-residual"]


def setup(s: systems.Structure, h=H, seed=0):
    w = weights.random_weights(h, seed)
    e = systems.neighbor_list(s, h.cutoff)
    pk = systems.packed_edges(len(s.positions), e, h.cutoff, h.cutoff_width)
    return w, pk, species_index(s.numbers, h.atomic_types)


def small_water(seed=0):
    """24 waters in a 9.3 A box: both species, about 25 neighbours an atom."""
    return systems.water_box(2, 6.2, seed=seed)


def test_attention_matches_c_oracle():
    s = small_water()
    w, pk, sp = setup(s, H)
    tix = om.TokenIndex(pk.off)
    rng = np.random.default_rng(3)
    N, E = len(sp), int(pk.off[-1])
    D, heads = 64, 4
    qkv = rng.standard_normal((N + E, 3 * D))
    cut = systems.cosine_cutoff(pk.dist, H.cutoff, H.cutoff_width)
    cf = np.zeros((N, tix.S))
    cf[:, 0] = 1.0
    for n in range(N):
        cf[n, 1:1 + pk.off[n + 1] - pk.off[n]] = cut[pk.off[n]:pk.off[n + 1]]
    mine = om.attention(torch.tensor(qkv), torch.tensor(cf), tix, heads, 1.0 / np.sqrt(D // heads)).numpy()
    ref, _ = oracle.attn_fwd(qkv, pk.off, cf, heads, D // heads, dtype=np.float64)
    assert np.abs(mine - ref).max() < 1e-12


def test_norms_match_torch():
    x = torch.randn(7, 48, dtype=torch.float64)
    w, b = torch.randn(48, dtype=torch.float64), torch.randn(48, dtype=torch.float64)
    assert torch.allclose(om.norm(x, w), torch.nn.functional.rms_norm(x, (48,), w, eps=om.RMS_EPS), atol=1e-13)
    assert torch.allclose(om.norm(x, w, b), torch.nn.functional.layer_norm(x, (48,), w, b, eps=om.LN_EPS), atol=1e-13)


@pytest.mark.parametrize("name", FAMILIES)
def test_edge_grad_central_differences(name):
    H = weights.MODELS[name]
    s = small_water(1)
    w, pk, sp = setup(s, H)
    comp = weights.random_composition(H)
    _, eg = om.evaluate(H, w, sp, pk, comp)
    rng = np.random.default_rng(0)
    E = int(pk.off[-1])
    hstep = 1e-5
    for k in rng.choice(E, 6, replace=False):
        for c in range(3):
            vals = []
            for sgn in (1, -1):
                v = torch.tensor(pk.vec[:E], dtype=torch.float64)
                v[k, c] += sgn * hstep
                pa, _ = om.evaluate(H, w, sp, pk, comp, grad=False, vec=v)
                vals.append(pa.sum())
            fd = (vals[0] - vals[1]) / (2 * hstep)
            assert abs(fd - eg[k, c]) < 1e-6 * max(1.0, abs(eg[k, c])), (k, c, fd, eg[k, c])


@pytest.mark.parametrize("name", FAMILIES)
def test_forces_central_differences(name):
    H = weights.MODELS[name]
    """forces = -dE/dr, by the fold of the edge gradients."""
    s = small_water(2)
    w, pk, sp = setup(s, H)
    _, eg = om.evaluate(H, w, sp, pk)
    f, _ = om.fold_forces(len(sp), pk, eg)
    hstep = 1e-5
    for a in (0, 5, 17):
        for c in range(3):
            vals = []
            for sgn in (1, -1):
                s2 = systems.Structure(s.positions.copy(), s.cell, s.numbers)
                s2.positions[a, c] += sgn * hstep
                w2, pk2, sp2 = setup(s2, H)
                pa, _ = om.evaluate(H, w, sp2, pk2, grad=False)
                vals.append(pa.sum())
            assert abs(-(vals[0] - vals[1]) / (2 * hstep) - f[a, c]) < 1e-6 * max(1.0, abs(f[a, c]))
    assert np.abs(f.sum(0)).max() < 1e-10


@pytest.mark.parametrize("name", FAMILIES)
def test_permutation_and_translation(name):
    H = weights.MODELS[name]
    s = small_water(3)
    w, pk, sp = setup(s, H)
    pa, eg = om.evaluate(H, w, sp, pk)
    f, _ = om.fold_forces(len(sp), pk, eg)
    perm = np.random.default_rng(1).permutation(len(sp))
    s2 = systems.Structure(s.positions[perm] + np.array([0.3, -1.1, 2.0]), s.cell, s.numbers[perm])
    _, pk2, sp2 = setup(s2, H)
    pa2, eg2 = om.evaluate(H, w, sp2, pk2)
    f2, _ = om.fold_forces(len(sp2), pk2, eg2)
    assert np.abs(pa2 - pa[perm]).max() < 1e-10
    assert np.abs(f2 - f[perm]).max() < 1e-9


@pytest.mark.parametrize("name", FAMILIES)
def test_supercell_extensive(name):
    H = weights.MODELS[name]
    cell = systems.diamond(1, jitter=0.0)
    sup = systems.diamond(2, jitter=0.0)
    w, pk, sp = setup(cell, H)
    w, pk2, sp2 = setup(sup, H)
    pa, _ = om.evaluate(H, w, sp, pk, grad=False)
    pa2, _ = om.evaluate(H, w, sp2, pk2, grad=False)
    # each supercell atom has the environment of its image in the cell (the two
    # sublattices differ: PET does not see inversion as a symmetry)
    assert np.abs(np.sort(pa2) - np.sort(np.tile(pa, 8))).max() < 1e-9 * np.abs(pa).max()
    assert np.ptp(pa) > 1e-3


@pytest.mark.parametrize("name", FAMILIES)
def test_fp32_close_to_fp64(name):
    H = weights.MODELS[name]
    s = small_water(4)
    w, pk, sp = setup(s, H)
    pa64, eg64 = om.evaluate(H, w, sp, pk)
    pa32, eg32 = om.evaluate(H, w, sp, pk, dtype=torch.float32)
    assert abs(pa32.sum() - pa64.sum()) < 1e-5 * abs(pa64.sum())
    assert np.abs(eg32 - eg64).max() < 1e-4 * np.abs(eg64).max()


def test_oracle_reduces_to_the_closed_form():
    """The oracle's composition where the mathematics fixes it: a PET with
    every block's output layers zeroed (tests/reduced_pet.py) has a closed-form
    energy -- species-embedding node features, edge features summed over the
    layers' compress maps, the readout of both."""
    from pet_kokkos_amd.model import structures_input
    from reduced_pet import closed_form_energy, reduced_weights
    h = weights.MODELS["tiny"]
    w = reduced_weights(h, 31)
    comp = weights.random_composition(h)
    for s in (systems.water_box(2, 6.2, seed=3), systems.diamond(1, jitter=0.05, seed=4)):
        x = structures_input(h, [s], "cpu")
        pa, _ = om.evaluate(h, w, x.species.numpy(), x.host, comp, grad=False)
        assert np.abs(pa - closed_form_energy(h, w, comp, s)).max() < 1e-10
