"""Element-wise parity checks shared by the tests.

The attention bar (outputs and gradients within 1e-5
relative) is applied to every element, with an absolute floor tied to the
scale of the element's row:

    |got - ref| <= RTOL * (|ref| + F_row)

F_row is the largest |ref| in the element's row: a token row of merged
[T, D] or qkv_adj [T, 3D], an atom's row of cf_seq_adj [N, S] or of cfh (all
heads and slots). An fp32 sum carries an error of order 1e-7 of the sum of
its terms' magnitudes, so an element much smaller than its row (a gradient
that nearly cancels) is held to its row's scale, not its own.

Two outputs are differences that can cancel to far below their row, so their
floor is the scale of the terms they are formed from (first-order rounding
error bounds, Euclidean norms through Cauchy-Schwarz):

- cfh[n, h, k] = sum_i dS_ik, dS_ik = A_ik (dP_ik - Dq_i), dP_ik = dO_i . v_k,
  Dq_i = dO_i . O_i. It cancels exactly for an atom whose only live key is its
  own token (the exact result is 0; fp32 leaves the rounding of the two dot
  products). Floor T[n, h, k] = sum_i A_ik |dO_i| (|v_k| + |O_i|), with A
  recomputed in float64; cf_seq_adj[n, k] = sum_h cfh / cf_k takes
  sum_h T / cf_k.
- the saved max logit m_i = max_k (scale q_i . k_k + log cf_k): floor
  scale |q_i| max_k |k_k|.
"""
from __future__ import annotations

import numpy as np

RTOL = 1e-5


def row_err(got, ref, width=None):
    """max over elements of |got - ref| / (|ref| + F_row), rows of `width`
    consecutive elements (default: the last axis)."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    if g.shape != r.shape:
        raise AssertionError(f"shape {g.shape} != {r.shape}")
    if r.size == 0:
        return 0.0
    w = width or r.shape[-1]
    g, r = g.reshape(-1, w), r.reshape(-1, w)
    floor = np.abs(r).max(1, keepdims=True)
    d = np.abs(g - r)
    den = np.abs(r) + floor
    bad = (den == 0) & (d > 0)
    if bad.any():
        return float("inf")
    with np.errstate(invalid="ignore", divide="ignore"):
        q = np.where(den > 0, d / np.where(den > 0, den, 1), 0.0)
    return float(q.max())


def slot_rows(off, S):
    """[N, S] token row of each (atom, slot), -1 past the atom's count."""
    off = np.asarray(off, np.int64)
    N = len(off) - 1
    cnt = np.minimum(np.diff(off) + 1, S)
    s = np.arange(S)[None, :]
    rows = np.where(s == 0, np.arange(N)[:, None], N + off[:-1, None] + s - 1)
    return np.where(s < cnt[:, None], rows, -1)


def term_scales(off, cf_seq, qkv, dmerged, H, hd, scale, chunk=256):
    """(T [N, H, S], q-scale [N, H, S]): the floors above, in float64."""
    cf = np.asarray(cf_seq, np.float64)
    N, S = cf.shape
    rows = slot_rows(off, S)
    D = H * hd
    x = np.asarray(qkv, np.float64)
    g = np.asarray(dmerged, np.float64)[:, :D]
    T = np.zeros((N, H, S))
    QS = np.zeros((N, H, S))
    with np.errstate(divide="ignore"):
        lcf = np.where(cf > 0, np.log(np.where(cf > 0, cf, 1.0)), -np.inf)
    for a in range(0, N, chunk):
        b = min(N, a + chunk)
        r = rows[a:b]
        valid = r >= 0
        rr = np.where(valid, r, 0)
        blk = lambda m, c0: np.where(valid[..., None, None], m[rr, c0:c0 + D].reshape(b - a, S, H, hd), 0.0)
        q, k, v = blk(x, 0), blk(x, D), blk(x, 2 * D)
        do = np.where(valid[..., None, None], g[rr].reshape(b - a, S, H, hd), 0.0)
        logit = scale * np.einsum("nihd,nkhd->nhik", q, k) + lcf[a:b, None, None, :]
        logit = np.where(valid[:, None, None, :], logit, -np.inf)
        live = valid & ((np.arange(S) == 0)[None, :] | (cf[a:b] > 0))  # queries with an output
        mx = np.max(np.where(np.isfinite(logit), logit, -1e300), axis=-1, keepdims=True)
        e = np.where(np.isfinite(logit), np.exp(logit - mx), 0.0)
        A = e / np.maximum(e.sum(-1, keepdims=True), 1e-300)
        A = np.where(live[:, None, :, None], A, 0.0)  # [n, h, i, k]
        O = np.einsum("nhik,nkhd->nihd", A, v)
        nq, nk, nv = (np.linalg.norm(t, axis=-1) for t in (q, k, v))  # [n, S, H]
        ng, no = np.linalg.norm(do, axis=-1), np.linalg.norm(O, axis=-1)
        T[a:b] = np.einsum("nhik,nih->nhk", A, ng * no) + np.einsum("nhik,nih->nhk", A, ng) * nv.transpose(0, 2, 1)
        QS[a:b] = scale * nq.transpose(0, 2, 1) * nk.max(1)[:, :, None]
    return T, QS


def floor_err(got, ref, floor):
    """max |got - ref| / (|ref| + max(F_row, floor)), rows = the first axis."""
    n = len(floor)
    g = np.asarray(got, np.float64).reshape(n, -1)
    r = np.asarray(ref, np.float64).reshape(n, -1)
    f = np.maximum(np.abs(r).max(1, keepdims=True), np.asarray(floor, np.float64).reshape(n, -1))
    d = np.abs(g - r)
    den = np.abs(r) + f
    if ((den == 0) & (d > 0)).any():
        return float("inf")
    return float(np.where(den > 0, d / np.where(den > 0, den, 1), 0.0).max()) if r.size else 0.0


def attention_errors(off, cf_seq, qkv, dmerged, H, hd, merged, qkv_adj, cf_seq_adj, cfh, ref, scale,
                     ml=None, ref_ml=None):
    """Per-tensor element-wise errors of (merged, qkv_adj, cf_seq_adj, cfh[,
    ml]) against ref = (merged, qkv_adj, cf_seq_adj, cfh); cfh in the
    reference's [N*S, H] layout, ml [N*H*S, 2]. Slots with no live query must
    hold the same (sentinel) statistics on both sides."""
    N, S = cf_seq.shape
    T, QS = term_scales(off, cf_seq, qkv, dmerged, H, hd, scale)
    cf = np.asarray(cf_seq, np.float64)
    ca_floor = np.where(cf > 0, T.sum(1) / np.where(cf > 0, cf, 1.0), 0.0)  # [N, S]
    out = dict(merged=row_err(merged, ref[0]), qkv_adj=row_err(qkv_adj, ref[1]),
               cf_seq_adj=floor_err(cf_seq_adj, ref[2], ca_floor),
               cfh=floor_err(np.asarray(cfh).reshape(N, S * H), np.asarray(ref[3]).reshape(N, S * H),
                             T.transpose(0, 2, 1).reshape(N, S * H)))
    if ml is not None:
        ml, ref_ml = np.asarray(ml, np.float64), np.asarray(ref_ml, np.float64)
        live = ref_ml[:, 1] > 0
        if not np.array_equal(ml[:, 1] > 0, live):
            raise AssertionError("live queries differ")
        if not np.array_equal(ml[~live].astype(np.float32), ref_ml[~live].astype(np.float32)):
            raise AssertionError("sentinel statistics differ")
        z = lambda a: np.where(live, a, 0.0).reshape(N * H, S)
        out["ml.max"] = floor_err(z(ml[:, 0]), z(ref_ml[:, 0]), QS.reshape(N * H, S))
        out["ml.invl"] = row_err(z(ml[:, 1]), z(ref_ml[:, 1]))
    return out
