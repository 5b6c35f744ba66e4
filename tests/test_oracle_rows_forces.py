"""Pins of the oracle's token norm, cf_seq and forces' edge term
(oracle/rows_forces_oracle.cpp), none of which retypes the oracle's formula:

- norm_rows / norm_rows_bwd: torch.nn.functional.rms_norm / layer_norm and
  their autograd in fp64 (a library, not the reference), closed forms of a
  constant row, the beta rule;
- cutoff derivatives: central differences of the cutoff values (fp64), the
  cosine closed form, and float-vs-double agreement of the reference's CutT
  evaluation;
- edge_grad: central differences of E(vec) = sum_k x4_adj_k . (vec_k, |vec_k|)
  + cutoff_total_k cf(|vec_k|), with cutoff_total_k built here from each
  edge's (atom, slot) -- which pins the slot mapping 1 + (k - off[n]);
- fold: forces = -dE/dr and virial = dE/d(strain) by central differences of a
  pair energy over a full directed neighbour list, which pins the signs, the
  reverse-edge term and the virial's index order;
- struct_sum and cf_seq: direct numpy sums / construction.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pet_kokkos_amd import systems


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


# ---- norms ----------------------------------------------------------------

@pytest.mark.parametrize("ln", [False, True])
@pytest.mark.parametrize("D", [64, 96, 256])
def test_norm_matches_torch_fp64(ln, D):
    rng = np.random.default_rng(D + ln)
    x = rng.standard_normal((37, D)) * 3 + 0.5
    w = rng.standard_normal(D)
    b = rng.standard_normal(D) if ln else None
    got = oracle.norm_rows(x, w, b, dtype=np.float64)
    xt = torch.from_numpy(x)
    if ln:
        ref = torch.nn.functional.layer_norm(xt, (D,), torch.from_numpy(w), torch.from_numpy(b), eps=1e-5)
    else:
        ref = torch.nn.functional.rms_norm(xt, (D,), torch.from_numpy(w), eps=float(np.finfo(np.float32).eps))
    assert rel(got, ref.numpy()) < 1e-13
    got32 = oracle.norm_rows(x, w, b, dtype=np.float32)
    assert rel(got32, ref.numpy()) < 2e-6


@pytest.mark.parametrize("ln", [False, True])
def test_norm_bwd_matches_torch_autograd(ln):
    D = 128
    rng = np.random.default_rng(3 + ln)
    x = rng.standard_normal((21, D)) * 2 + 0.3
    w = rng.standard_normal(D)
    b = rng.standard_normal(D) if ln else None
    g = rng.standard_normal((21, D))
    xt = torch.from_numpy(x).requires_grad_(True)
    if ln:
        y = torch.nn.functional.layer_norm(xt, (D,), torch.from_numpy(w), torch.from_numpy(b), eps=1e-5)
    else:
        y = torch.nn.functional.rms_norm(xt, (D,), torch.from_numpy(w), eps=float(np.finfo(np.float32).eps))
    (y * torch.from_numpy(g)).sum().backward()
    got = oracle.norm_rows_bwd(g, x, w, ln, dtype=np.float64)
    assert rel(got, xt.grad.numpy()) < 1e-12
    got32 = oracle.norm_rows_bwd(g, x, w, ln, dtype=np.float32)
    assert rel(got32, xt.grad.numpy()) < 1e-5
    # beta: scaled accumulation onto in_adj
    prev = rng.standard_normal((21, D))
    acc = oracle.norm_rows_bwd(g, x, w, ln, beta=0.5, in_adj=prev, dtype=np.float64)
    assert rel(acc, 0.5 * prev + xt.grad.numpy()) < 1e-12


def test_norm_constant_row_closed_forms():
    D = 64
    w = np.linspace(0.5, 1.5, D)
    b = np.linspace(-1, 1, D)
    c = 2.5
    x = np.full((1, D), c)
    eps = float(np.finfo(np.float32).eps)
    rms = oracle.norm_rows(x, w, None, dtype=np.float64)
    assert rel(rms[0], c / np.sqrt(c * c + eps) * w) < 1e-15
    lnr = oracle.norm_rows(x, w, b, dtype=np.float64)
    assert np.array_equal(lnr[0], b)  # x - mean = 0 exactly


# ---- cutoff derivatives -------------------------------------------------------

@pytest.mark.parametrize("kind", [0, 1, 2])
def test_cutoff_derivative_is_the_values_slope(kind):
    rc, w = 4.5, 0.5
    d = np.linspace(3.95, 4.55, 61)[1:-1]
    d = d[np.abs((d - (rc - w)) / w - np.round((d - (rc - w)) / w)) > 1e-3]  # off the taper's ends
    h = 1e-6
    vp, _ = oracle.cutoff(d + h, rc, w, kind, f64=True)
    vm, _ = oracle.cutoff(d - h, rc, w, kind, f64=True)
    _, dd = oracle.cutoff(d, rc, w, kind, f64=True)
    fd = (vp - vm) / (2 * h)
    assert np.abs(dd - fd).max() < 1e-6 * max(1.0, np.abs(fd).max())
    # the reference's evaluation (transcendentals in float) agrees to float precision
    _, dd32 = oracle.cutoff(d, rc, w, kind, f64=False)
    assert np.abs(dd32 - dd).max() < 2e-5 * max(1.0, np.abs(dd).max())


def test_cosine_cutoff_closed_form():
    rc, w = 4.5, 0.5
    d = np.array([3.9, 4.0, 4.1, 4.25, 4.4, 4.5, 4.6])
    v, dd = oracle.cutoff(d, rc, w, 1, f64=True)
    x = np.clip((d - (rc - w)) / w, 0, 1)
    assert np.allclose(v, 0.5 * (1 + np.cos(np.pi * x)), atol=1e-15)
    inside = (x > 0) & (x < 1)
    assert np.allclose(dd[inside], -0.5 * np.pi * np.sin(np.pi * x[inside]) / w, atol=1e-13)
    assert np.all(dd[~inside] == 0.0)


# ---- the edge term --------------------------------------------------------------

def _small_edges(seed=0, n_dead=0):
    s = systems.diamond(1, jitter=0.05, seed=seed)  # 8 atoms, cutoff 3.0: a few neighbours each
    e = systems.neighbor_list(s, 3.0)
    pk = systems.packed_edges(len(s.positions), e, 3.0, 0.5)
    return s, e, pk


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_edge_grad_is_dE_dvec(kind):
    s, e, pk = _small_edges(kind)
    N, E = len(s.positions), len(pk.center)
    S = int(np.diff(pk.off).max()) + 1
    rng = np.random.default_rng(10 + kind)
    x4 = rng.standard_normal((E, 4)).astype(np.float32)
    cadj = rng.standard_normal(E).astype(np.float32)
    csa = rng.standard_normal((N, S)).astype(np.float32)
    rc, w = 3.0, 0.8
    pcut = np.full(E, rc)
    # cutoff_total of edge k from its own (atom, slot), built independently here
    slot = np.arange(E) - pk.off[pk.center]
    ctot = (cadj + csa[pk.center, 1 + slot]).astype(np.float32).astype(np.float64)

    def energy(vec):
        d = np.linalg.norm(vec, axis=1)
        cf, _ = oracle.cutoff(d, pcut, w, kind, f64=True)
        return float(np.sum(x4[:, :3].astype(np.float64) * vec) + np.sum(x4[:, 3] * d) + np.sum(ctot * cf))

    got = oracle.edge_grad(pk.off, pk.center, x4, cadj, csa, pk.vec, pk.dist, pcut, w, kind)
    fd = np.zeros_like(pk.vec)
    h = 1e-6
    for k in range(E):
        for c in range(3):
            vp, vm = pk.vec.copy(), pk.vec.copy()
            vp[k, c] += h
            vm[k, c] -= h
            fd[k, c] = (energy(vp) - energy(vm)) / (2 * h)
    assert rel(got, fd) < 1e-5


def test_edge_grad_dead_rows_and_no_cutoff_adj():
    s, e, pk = _small_edges(1)
    N, E = len(s.positions), len(pk.center)
    S = int(np.diff(pk.off).max()) + 1
    rng = np.random.default_rng(2)
    x4 = rng.standard_normal((E + 5, 4)).astype(np.float32)
    csa = rng.standard_normal((N, S)).astype(np.float32)
    pad = lambda a, v: np.concatenate([a, np.full((5,) + a.shape[1:], v, dtype=a.dtype)])
    g = oracle.edge_grad(pk.off, pad(pk.center, 0), x4, None, csa, pad(pk.vec, 1.0), pad(pk.dist, 1.0),
                         pad(pk.pcut, 3.0), 0.5, 1)
    assert np.all(g[E:] == 0.0)
    g0 = oracle.edge_grad(pk.off, pk.center, x4[:E], np.zeros(E, np.float32), csa, pk.vec, pk.dist, pk.pcut, 0.5, 1)
    assert np.array_equal(g[:E], g0)


# ---- the fold -----------------------------------------------------------------

def _pair_energy_and_grad(vec):
    """phi(v) = sum_k exp(-|v|^2 / 4) (1 + 0.3 v_x) and its gradient per edge."""
    d2 = np.einsum("ij,ij->i", vec, vec)
    a = np.exp(-d2 / 4.0)
    e = np.sum(a * (1 + 0.3 * vec[:, 0]))
    g = (-0.5 * vec) * (a * (1 + 0.3 * vec[:, 0]))[:, None]
    g[:, 0] += 0.3 * a
    return e, g


def test_fold_forces_and_virial_by_finite_differences():
    s = systems.diamond(1, jitter=0.08, seed=5)
    x0, cell = s.positions.copy(), s.cell.copy()
    rc = 3.0
    e = systems.neighbor_list(s, rc)
    pk = systems.packed_edges(len(x0), e, rc)
    assert np.all(pk.reverse >= 0)
    N = len(x0)

    def energy_of(x, c):
        vec = x[pk.neigh] + e.shift @ c - x[pk.center]
        return _pair_energy_and_grad(vec)[0]

    _, g = _pair_energy_and_grad(pk.vec)
    forces, vir = oracle.fold(N, pk.off, pk.reverse, pk.vec, g, scale=1.0)
    # forces = -dE/dr: with every edge's reverse present, F_i = sum_k g_k - g_rev(k)
    # over i's edges counts each pair from both ends, E sums both directions
    h = 1e-6
    fd = np.zeros((N, 3))
    for i in range(N):
        for c in range(3):
            xp, xm = x0.copy(), x0.copy()
            xp[i, c] += h
            xm[i, c] -= h
            fd[i, c] = -(energy_of(xp, cell) - energy_of(xm, cell)) / (2 * h)
    assert rel(forces, fd) < 1e-6
    # virial: W_ab = dE/d eps_ab for r -> r (1 + eps), cell -> cell (1 + eps)
    W = vir.sum(axis=0).reshape(3, 3)
    fdw = np.zeros((3, 3))
    for a in range(3):
        for b in range(3):
            ep = np.eye(3)
            em = np.eye(3)
            ep[a, b] += h
            em[a, b] -= h
            fdw[a, b] = (energy_of(x0 @ ep, cell @ ep) - energy_of(x0 @ em, cell @ em)) / (2 * h)
    assert rel(W, fdw) < 1e-6
    # scale multiplies both
    f2, v2 = oracle.fold(N, pk.off, pk.reverse, pk.vec, g, scale=-2.0)
    assert np.allclose(f2, -2 * forces, rtol=0, atol=1e-14) and np.allclose(v2, -2 * vir, rtol=0, atol=1e-14)


def test_fold_partnerless_edges_and_neighbour_only_atoms():
    # atom 2 owns no edges (n_centres = 2 of N = 3); edge 1 has no reverse
    off = np.array([0, 2, 3], np.int32)
    rev = np.array([2, -1, 0], np.int32)
    vec = np.array([[1.0, 0, 0], [0, 1.0, 0], [-1.0, 0, 0]])
    g = np.array([[1.0, 2, 3], [4.0, 5, 6], [7.0, 8, 9]])
    f, v = oracle.fold(3, off, rev, vec, g)
    assert np.allclose(f[0], g[0] + g[1] - g[2])
    assert np.allclose(f[1], g[2] - g[0])
    assert np.all(f[2] == 0) and np.all(v[2] == 0)
    assert np.allclose(v[0].reshape(3, 3), np.outer(vec[0], g[0]) + np.outer(vec[1], g[1]))


def test_struct_sum_and_cf_seq():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((10, 9))
    soff = np.array([0, 3, 3, 10], np.int32)
    out = oracle.struct_sum(soff, x)
    assert np.allclose(out, [x[0:3].sum(0), np.zeros(9), x[3:10].sum(0)], rtol=0, atol=1e-14)
    assert np.allclose(oracle.struct_sum(soff, x, out, acc=True), 2 * out, rtol=0, atol=1e-14)
    off = np.array([0, 2, 2, 5], np.int32)
    cut = np.array([0.5, 0.25, 0.9, 0.8, 0.7], np.float32)
    cf = oracle.cf_seq(off, cut, 5)
    assert np.array_equal(cf, np.array([[1, 0.5, 0.25, 0, 0], [1, 0, 0, 0, 0], [1, 0.9, 0.8, 0.7, 0]], np.float32))
