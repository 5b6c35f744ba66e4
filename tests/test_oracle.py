"""Pins of the CPU oracle (oracle/attention_oracle.cpp), run without a GPU.

The reference cannot be built or imported here (its build fetches Kokkos and
more at configure time; it has no Python implementation of the path), and its
own tests hold no attention-level vectors. So each oracle function is pinned
by checks a plausible slip would fail:

  fwd, bwd    golden vectors of an independent float64 brute force (full
              softmax + torch.autograd, tests/golden/make_golden.py), with the
              fp64 twin to 1e-11 and the fp32 build to 1e-5, per tensor and
              element by element (tests/parity.py's row-floor rule); closed forms (one
              token; zero queries); torch's scaled_dot_product_attention when
              every cf is 1; central differences of the fp64 twin; invariants
              (sum_k cfh = 0, cf scale invariance, permutation equivariance);
  cf adjoint  the golden cf_seq_adj (= d loss / d cf) and the accumulate rule;
  zero_dead   dead rows zero, live rows untouched;
  linear      numpy float64 matmul.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

import oracle
from parity import attention_errors
from pet_kokkos_amd import systems

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "attn_*.npz")))


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def random_case(counts, H, hd, seed=0, cf_kind="random", extra=0, temperature=1.0):
    base = systems.tokens_from_counts(counts, seed=seed, cf_kind=cf_kind)
    tk = systems.tokens_from_counts(counts, seed=seed, cf_kind=cf_kind, slots=base.slots + extra)
    rng = np.random.default_rng(seed + 7)
    D = H * hd
    qkv = rng.standard_normal((tk.n_rows, 3 * D))
    dm = rng.standard_normal((tk.n_rows, D))
    return tk, qkv, dm


def test_oracle_builds():
    assert os.path.exists(oracle.build())


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
@pytest.mark.parametrize("dtype,tol", [(np.float64, 1e-11), (np.float32, 1e-5)])
def test_golden(path, dtype, tol):
    g = np.load(path)
    H, hd, temp = int(g["heads"]), int(g["head_dim"]), float(g["temperature"])
    merged, ml = oracle.attn_fwd(g["qkv"], g["off"], g["cf_seq"], H, hd, temp, dtype=dtype)
    assert rel(merged, g["merged"]) < tol
    live = g["ml"][:, 1] > 0
    assert np.array_equal(ml[:, 1] > 0, live)
    assert np.all(ml[~live, 0] == np.float32(-1e30)) if dtype == np.float32 else np.all(ml[~live, 0] == -1e30)
    assert rel(ml[live, 0], g["ml"][live, 0]) < tol
    assert rel(ml[live, 1], g["ml"][live, 1]) < tol
    qkv_adj, cf_adj, cfh = oracle.attn_bwd(g["qkv"], g["off"], g["dmerged"], merged, ml, g["cf_seq"], H, hd, temp,
                                           dtype=dtype)
    assert rel(qkv_adj, g["qkv_adj"]) < tol
    assert rel(cfh, g["cfh"]) < tol
    assert rel(cf_adj, g["cf_seq_adj"]) < tol
    # and element by element, each held to its row's scale (tests/parity.py)
    errs = attention_errors(g["off"], g["cf_seq"], g["qkv"], g["dmerged"], H, hd, merged, qkv_adj, cf_adj, cfh,
                            (g["merged"], g["qkv_adj"], g["cf_seq_adj"], g["cfh"]), float(g["scale"]),
                            ml.astype(np.float32) if dtype == np.float32 else ml, g["ml"])
    for k, v in errs.items():
        assert v < tol, (k, v)


def test_single_token_closed_form():
    # cnt = 1: out = v0; dQ = dK = 0, dV = dO; cfh = 0 (reference Forward/Queries/Keys with one key).
    tk, qkv, dm = random_case([0, 0, 0], 2, 16)
    merged, ml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, 16, dtype=np.float64)
    assert np.allclose(merged, qkv[:, 64:96], rtol=0, atol=1e-15)
    assert np.allclose(ml[ml[:, 1] > 0, 1], 1.0)
    qa, ca, cfh = oracle.attn_bwd(qkv, tk.off, dm, merged, ml, tk.cf_seq, 2, 16, dtype=np.float64)
    assert np.all(qa[:, :64] == 0)
    assert np.allclose(qa[:, 64:], dm, atol=1e-15)
    assert np.all(cfh == 0) and np.all(ca == 0)


def test_zero_queries_closed_form():
    # q = 0: weights cf_k / sum cf, out = sum_k cf_k v_k / sum_k cf_k for live queries.
    tk, qkv, _ = random_case([5, 9, 17], 2, 32, seed=3, cf_kind="zeros")
    D = 64
    qkv[:, :D] = 0
    merged, _ = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, 32, dtype=np.float64)
    for n in range(tk.n_atoms):
        rows = tk.rows(n)
        cf = tk.cf_seq[n, :len(rows)].astype(np.float64)
        expect = (cf[:, None] * qkv[rows, 2 * D:]).sum(0) / cf.sum()
        for s, r in enumerate(rows):
            if s == 0 or cf[s] > 0:
                assert np.allclose(merged[r], expect, rtol=1e-13, atol=1e-13)
            else:
                assert np.all(merged[r] == 0)


def test_all_cf_one_is_sdpa():
    # All cf = 1: plain scaled dot-product attention per atom and head.
    tk, qkv, _ = random_case([12, 30, 3], 3, 16, seed=5, cf_kind="ones")
    H, hd = 3, 16
    D = H * hd
    merged, _ = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, H, hd, dtype=np.float64)
    sc = oracle.scale(hd)
    for n in range(tk.n_atoms):
        rows = tk.rows(n)
        x = torch.tensor(qkv[rows], dtype=torch.float64)
        q = x[:, :D].reshape(-1, H, hd).transpose(0, 1)
        k = x[:, D:2 * D].reshape(-1, H, hd).transpose(0, 1)
        v = x[:, 2 * D:].reshape(-1, H, hd).transpose(0, 1)
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=sc)
        assert np.allclose(merged[rows], o.transpose(0, 1).reshape(len(rows), D).numpy(), rtol=1e-12, atol=1e-12)


def test_finite_differences():
    # d loss / d qkv and d loss / d cf of the fp64 twin against central differences,
    # loss = sum(merged * dm), the sweep of h as in the reference's tests/test_fd.cpp.
    tk, qkv, dm = random_case([6, 3, 10], 2, 16, seed=11)
    H, hd = 2, 16

    def loss(q, cf):
        m, _ = oracle.attn_fwd(q, tk.off, cf, H, hd, dtype=np.float64)
        return float((m * dm).sum())

    cf = tk.cf_seq.astype(np.float64)
    merged, ml = oracle.attn_fwd(qkv, tk.off, cf, H, hd, dtype=np.float64)
    qa, ca, _ = oracle.attn_bwd(qkv, tk.off, dm, merged, ml, cf, H, hd, dtype=np.float64)
    rng = np.random.default_rng(0)
    for _ in range(25):
        r, c = rng.integers(tk.n_rows), rng.integers(3 * H * hd)
        best = np.inf
        for h in (1e-3, 1e-4, 1e-5):
            qp, qm = qkv.copy(), qkv.copy()
            qp[r, c] += h
            qm[r, c] -= h
            fd = (loss(qp, cf) - loss(qm, cf)) / (2 * h)
            best = min(best, abs(fd - qa[r, c]))
        assert best < 1e-6 * max(1.0, abs(qa[r, c]))
    for n in range(tk.n_atoms):
        for k in range(1, int(tk.off[n + 1] - tk.off[n]) + 1):
            h = 1e-5
            cp, cm = cf.copy(), cf.copy()
            cp[n, k] += h
            cm[n, k] -= h
            fd = (loss(qkv, cp) - loss(qkv, cm)) / (2 * h)
            assert abs(fd - ca[n, k]) < 1e-5 * max(1.0, abs(ca[n, k]))


def test_invariants():
    tk, qkv, dm = random_case([20, 33, 8, 1], 2, 32, seed=21, cf_kind="zeros")
    H, hd = 2, 32
    D = H * hd
    cf = tk.cf_seq.astype(np.float64)
    merged, ml = oracle.attn_fwd(qkv, tk.off, cf, H, hd, dtype=np.float64)
    qa, ca, cfh = oracle.attn_bwd(qkv, tk.off, dm, merged, ml, cf, H, hd, dtype=np.float64)
    # sum_k cfh[n, k, h] = 0: sum_k A_ik (dP_ik - Dq_i) = 0 for every live query.
    assert np.abs(cfh.reshape(tk.n_atoms, tk.slots, H).sum(1)).max() < 1e-12
    # every cf of an atom times a constant: the output is unchanged.
    m2, _ = oracle.attn_fwd(qkv, tk.off, cf * 3.7, H, hd, dtype=np.float64)
    assert np.allclose(m2, merged, rtol=1e-12, atol=1e-12)
    # a permutation of atom 0's edge slots permutes its rows and cf slots.
    n = 0
    cnt = int(tk.off[1] - tk.off[0])
    perm = np.random.default_rng(1).permutation(cnt)
    rows = tk.n_atoms + tk.off[0] + np.arange(cnt)
    q2, dm2, cf2 = qkv.copy(), dm.copy(), cf.copy()
    q2[rows] = qkv[rows[perm]]
    dm2[rows] = dm[rows[perm]]
    cf2[n, 1:1 + cnt] = cf[n, 1 + perm]
    m3, ml3 = oracle.attn_fwd(q2, tk.off, cf2, H, hd, dtype=np.float64)
    assert np.allclose(m3[rows], merged[rows[perm]], rtol=1e-12, atol=1e-12)
    assert np.allclose(m3[n], merged[n], rtol=1e-12, atol=1e-12)
    qa3, ca3, _ = oracle.attn_bwd(q2, tk.off, dm2, m3, ml3, cf2, H, hd, dtype=np.float64)
    assert np.allclose(qa3[rows], qa[rows[perm]], rtol=1e-10, atol=1e-12)
    assert np.allclose(ca3[n, 1:1 + cnt], ca[n, 1 + perm], rtol=1e-10, atol=1e-12)
    # a cf = 0 query outputs zeros and gets no gradient; a cf = 0 key is invisible.
    for n in range(tk.n_atoms):
        for s in range(1, int(tk.off[n + 1] - tk.off[n]) + 1):
            if cf[n, s] == 0:
                r = tk.n_atoms + tk.off[n] + s - 1
                assert np.all(merged[r] == 0) and np.all(qa[r] == 0) and ca[n, s] == 0
    _ = D


def test_cf_adjoint_accumulates():
    tk, qkv, dm = random_case([10, 4], 2, 16, seed=2)
    merged, ml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, 16)
    _, ca, _ = oracle.attn_bwd(qkv, tk.off, dm, merged, ml, tk.cf_seq, 2, 16)
    start = np.random.default_rng(0).standard_normal(ca.shape).astype(np.float32)
    _, ca2, _ = oracle.attn_bwd(qkv, tk.off, dm, merged, ml, tk.cf_seq, 2, 16, cf_seq_adj=start)
    assert np.array_equal(ca2, (start + ca).astype(np.float32)) or rel(ca2, start + ca) < 1e-6


def test_zero_dead():
    counts = [5, 7]
    tk = systems.tokens_from_counts(counts, seed=0)
    T = tk.n_rows + 6  # six dead capacity rows
    rng = np.random.default_rng(0)
    qkv = rng.standard_normal((T, 96)).astype(np.float32)
    dm = rng.standard_normal((T, 32)).astype(np.float32)
    m, ml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, 16, dead=True)
    assert np.all(m[tk.n_rows:] == 0)
    qa, _, _ = oracle.attn_bwd(qkv, tk.off, dm, m, ml, tk.cf_seq, 2, 16, dead=True)
    assert np.all(qa[tk.n_rows:] == 0)
    m2, _ = oracle.attn_fwd(qkv[:tk.n_rows], tk.off, tk.cf_seq, 2, 16)
    assert np.array_equal(m[:tk.n_rows], m2)


def test_linear_matches_numpy():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((37, 24)).astype(np.float32)
    W = rng.standard_normal((40, 24)).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    y0 = rng.standard_normal((37, 40)).astype(np.float32)
    y = oracle.linear(x, W, b, beta=0.5, out=y0)
    ref = x.astype(np.float64) @ W.T.astype(np.float64) + b + 0.5 * y0
    assert rel(y, ref) < 1e-6
    g = rng.standard_normal((37, 40)).astype(np.float32)
    xa0 = rng.standard_normal((37, 24)).astype(np.float32)
    xa = oracle.linear_bwd(g, W, beta=1.0, out=xa0)
    assert rel(xa, g.astype(np.float64) @ W.astype(np.float64) + xa0) < 1e-6


def test_repeatable_bitwise():
    tk, qkv, dm = random_case([30, 12, 45], 4, 16, seed=9)
    a = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 4, 16)
    b = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 4, 16)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
