"""Checks of the whole evaluation's composition that the mathematics fixes,
independent of the model oracle (oracle/pet_model.py):

- a reduced PET: with every attention output linear, centre expansion, MLP
  output layer and combination output layer zeroed (weights and biases), the
  feedforward featurizer's layers leave the node features at their species
  embedding and the edge features follow ie <- ie + compress_L(ie); the energy
  is then a closed form (the readout of those), computed here in numpy float64
  and differentiated by central differences;
- with the attention output linears' weights zeroed, the energy and forces do
  not depend on the attention's input linears at all (bit for bit);
- a structure evaluated inside a batch equals the same structure alone
  (configs[4]'s full 32-structure, 11,392-atom batch), to fp32 roundings;
- a periodic supercell's per-atom energies are the cell's (extensivity).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from pet_kokkos_amd import systems, weights
from pet_kokkos_amd.model import PetModel, ef_workload, structures_input
from reduced_pet import closed_form_energy, reduced_weights

pytestmark = pytest.mark.gpu


def test_reduced_model_closed_form(device):
    h = weights.MODELS["tiny"]
    w = reduced_weights(h, 31)
    comp = weights.random_composition(h)
    sts = [systems.water_box(2, 6.2, seed=3), systems.diamond(1, jitter=0.05, seed=4)]
    print("[gpu] reduced PET against its closed form", flush=True)
    got = PetModel(h, w, comp).compute(structures_input(h, sts, device), forces=True)
    torch.cuda.synchronize()
    pa = got["per_atom"].cpu().numpy()
    F = got["forces"].cpu().numpy()
    a = 0
    for s in sts:
        n = len(s.positions)
        ref = closed_form_energy(h, w, comp, s)
        err = np.abs(pa[a:a + n] - ref).max()
        print(f"    per-atom energy error {err:.2e} (largest |value| {np.abs(ref).max():.3g})", flush=True)
        assert err <= 1e-5 * np.abs(ref).max()
        assert abs(pa[a:a + n].sum() - ref.sum()) <= 1e-6 * np.abs(ref).sum()
        # forces: central differences of the closed form
        fd = np.zeros((n, 3))
        step = 1e-5
        for i in range(n):
            for c in range(3):
                sp_, sm = dataclasses.replace(s), dataclasses.replace(s)
                sp_.positions = s.positions.copy()
                sm.positions = s.positions.copy()
                sp_.positions[i, c] += step
                sm.positions[i, c] -= step
                fd[i, c] = -(closed_form_energy(h, w, comp, sp_).sum() - closed_form_energy(h, w, comp, sm).sum()) / (
                    2 * step)
        ferr = np.abs(F[a:a + n] - fd).max()
        print(f"    forces error {ferr:.2e} eV/A (largest {np.abs(fd).max():.3g})", flush=True)
        assert ferr <= 5e-5
        a += n


def test_attention_enters_only_through_its_output_linear(device):
    h = weights.MODELS["tiny"]
    w = weights.random_weights(h, 32)
    for k in w:
        if k.endswith(".attention.output_linear.weight"):
            w[k] = np.zeros_like(w[k])
    w2 = dict(w)
    rng = np.random.default_rng(5)
    for k in w:
        if ".attention.input_linear." in k:
            w2[k] = rng.standard_normal(w[k].shape)
    comp = weights.random_composition(h)
    x = structures_input(h, [systems.water_box(2, 6.2, seed=7)], device)
    a = PetModel(h, w, comp).compute(x, forces=True, edge_grad=True)
    a = {k: v.clone() for k, v in a.items()}
    b = PetModel(h, w2, comp).compute(x, forces=True, edge_grad=True)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_batched_equals_alone_c5(device):
    h, w, comp, sts = ef_workload("c5")
    m = PetModel(h, w, comp)
    print(f"[gpu] c5 batch of {len(sts)} structures against four of them alone", flush=True)
    x = structures_input(h, sts, device)
    got = m.compute(x, forces=True)
    torch.cuda.synchronize()
    pa_all = got["per_atom"].cpu().numpy()
    f_all = got["forces"].cpu().numpy()
    e_all = got["energy"].cpu().numpy()
    soff = x.struct_off.cpu().numpy()
    del x, got
    for k in (0, 1, 16, 31):
        alone = m.compute(structures_input(h, [sts[k]], device), forces=True)
        torch.cuda.synchronize()
        a, b = soff[k], soff[k + 1]
        pa, f = alone["per_atom"].cpu().numpy(), alone["forces"].cpu().numpy()
        de = abs(float(alone["energy"][0]) - e_all[k]) / abs(e_all[k])
        dpa = np.abs(pa - pa_all[a:b]).max() / np.abs(pa).max()
        df = np.abs(f - f_all[a:b]).max()
        print(f"    structure {k} ({b - a} atoms): energy {de:.1e} relative, per-atom {dpa:.1e}, forces {df:.1e} eV/A",
              flush=True)
        # the batch's large dense products run on the split-product kernel and
        # a lone structure's on rocBLAS and the short-K kernel (the default
        # model_gemm 6): the two
        # differ by fp32 roundings (on C2-size products a per-atom energy
        # differs from the float64 oracle by about 1e-6 of the largest;
        # measured here up to 5.3e-5 eV/A on forces). With every product on
        # this library's kernels the two are the same bits
        # (test_batched_equals_alone_c5_own_kernels)
        assert de <= 5e-6 and dpa <= 5e-6 and df <= 1e-4


def test_batched_equals_alone_c5_own_kernels(device):
    """Under PET_OPT_MODEL_GEMM 5 every dense product runs on this library's
    kernels, whose results for a row do not depend on the other rows; the
    attention, norms and folds are per item, row or atom. So a structure's
    per-atom energies and forces in the 32-structure C5 batch are the same
    bits as the structure's alone, and its energy (a per-structure sum of the
    same per-atom values) too."""
    from pet_kokkos_amd import _lib
    h, w, comp, sts = ef_workload("c5")
    old = _lib.get_option("model_gemm")
    _lib.set_option("model_gemm", 5)
    try:
        m = PetModel(h, w, comp)
        print(f"[gpu] c5 batch of {len(sts)} structures against four of them alone, model_gemm 5", flush=True)
        x = structures_input(h, sts, device)
        got = m.compute(x, forces=True)
        torch.cuda.synchronize()
        pa_all, f_all, e_all = (got[k].cpu().numpy() for k in ("per_atom", "forces", "energy"))
        soff = x.struct_off.cpu().numpy()
        del x, got
        for k in (0, 1, 16, 31):
            alone = m.compute(structures_input(h, [sts[k]], device), forces=True)
            torch.cuda.synchronize()
            a, b = soff[k], soff[k + 1]
            pa, f = alone["per_atom"].cpu().numpy(), alone["forces"].cpu().numpy()
            e = float(alone["energy"][0])
            print(f"    structure {k} ({b - a} atoms): per-atom max diff {np.abs(pa - pa_all[a:b]).max():.1e}, "
                  f"forces {np.abs(f - f_all[a:b]).max():.1e}, energy {abs(e - e_all[k]):.1e}", flush=True)
            assert np.array_equal(pa, pa_all[a:b]) and np.array_equal(f, f_all[a:b]) and e == e_all[k]
    finally:
        _lib.set_option("model_gemm", old)


def test_supercell_is_extensive(device):
    h = weights.MODELS["tiny"]
    w = weights.random_weights(h, 33)
    comp = weights.random_composition(h)
    cell = systems.diamond(2, jitter=0.03, seed=8)
    n = len(cell.positions)
    shifts = np.array([[i, j, k] for i in range(2) for j in range(2) for k in range(2)], dtype=np.float64)
    pos = (cell.positions[None, :, :] + (shifts @ cell.cell)[:, None, :]).reshape(-1, 3)
    sup = systems.Structure(pos, 2 * cell.cell, np.tile(cell.numbers, 8))
    got = PetModel(h, w, comp).compute(structures_input(h, [cell, sup], device), forces=True)
    torch.cuda.synchronize()
    pa = got["per_atom"].cpu().numpy()
    f = got["forces"].cpu().numpy()
    base, big = pa[:n], pa[n:].reshape(8, n)
    fb, fs = f[:n], f[n:].reshape(8, n, 3)
    print(f"[gpu] supercell: per-atom {np.abs(big - base).max():.1e}, forces {np.abs(fs - fb).max():.1e}", flush=True)
    assert np.abs(big - base).max() <= 1e-6 * np.abs(base).max()
    assert np.abs(fs - fb).max() <= 2e-5
    assert abs(got["energy"][1].item() - 8 * got["energy"][0].item()) <= 1e-6 * abs(8 * got["energy"][0].item())
