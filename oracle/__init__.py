"""TEST INFRASTRUCTURE ONLY: numpy bindings of the CPU oracle
(attention_oracle.cpp, a restatement of the reference's host attention path;
rows_forces_oracle.cpp, of its token norm, cf_seq and the forces' edge term).

Imported by tests/, by __graft_entry__.smoke() as the checker, and by bench.py's
cpu_baseline leg -- never by the product package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_attn.so")


class Shape(ctypes.Structure):
    _fields_ = [
        ("n_atoms", ctypes.c_int),
        ("n_rows", ctypes.c_int),
        ("slots", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("dead", ctypes.c_int),
        ("scale", ctypes.c_float),
    ]


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def scale(head_dim: int, temperature: float = 1.0) -> float:
    """float(1 / (sqrt(double(hd)) * T)), src/attention.cpp:1525."""
    return float(np.float32(1.0 / (np.sqrt(np.float64(head_dim)) * temperature)))


def shape(N, T, S, heads, head_dim, temperature=1.0, dead=False, sc=None):
    return Shape(N, T, S, heads, head_dim, int(dead), scale(head_dim, temperature) if sc is None else sc)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


def attn_fwd(qkv, off, cf_seq, heads, head_dim, temperature=1.0, N=None, dead=False, dtype=np.float32, sc=None):
    """(merged [T, D], ml [N*H*S, 2]) of the reference's Forward (src/attention.cpp:205-266)."""
    lib = load()
    qkv, cf_seq = _c(qkv, dtype), _c(cf_seq, dtype)
    off = _c(off, np.int32)
    T = qkv.shape[0]
    N = len(off) - 1 if N is None else N
    S = cf_seq.shape[1]
    D = heads * head_dim
    merged = np.zeros((T, D), dtype=dtype)
    ml = np.zeros((N * heads * S, 2), dtype=dtype)
    sh = shape(N, T, S, heads, head_dim, temperature, dead, sc)
    fn = lib.oracle_attn_fwd_f32 if dtype == np.float32 else lib.oracle_attn_fwd_f64
    fn(ctypes.byref(sh), _p(qkv), ctypes.c_int64(qkv.shape[1]), _p(off), _p(cf_seq), ctypes.c_int64(S), _p(merged),
       ctypes.c_int64(D), _p(ml))
    return merged, ml


def attn_bwd(qkv, off, dmerged, merged, ml, cf_seq, heads, head_dim, temperature=1.0, cf_seq_adj=None, N=None,
             dead=False, dtype=np.float32, sc=None):
    """(qkv_adj [T, 3D], cf_seq_adj [N, S], cfh [N*S, H]) of the reference's
    Queries, Keys and attn_bwd_cf (src/attention.cpp:1560-1697, :1829-1838)."""
    lib = load()
    qkv, dmerged, merged, ml, cf_seq = (_c(a, dtype) for a in (qkv, dmerged, merged, ml, cf_seq))
    off = _c(off, np.int32)
    T = qkv.shape[0]
    N = len(off) - 1 if N is None else N
    S = cf_seq.shape[1]
    D = heads * head_dim
    qkv_adj = np.zeros((T, 3 * D), dtype=dtype)
    cfh = np.zeros((N * S, heads), dtype=dtype)
    cf_seq_adj = np.zeros((N, S), dtype=dtype) if cf_seq_adj is None else _c(cf_seq_adj, dtype).copy()
    sh = shape(N, T, S, heads, head_dim, temperature, dead, sc)
    fn = lib.oracle_attn_bwd_f32 if dtype == np.float32 else lib.oracle_attn_bwd_f64
    fn(ctypes.byref(sh), _p(qkv), ctypes.c_int64(3 * D), _p(off), _p(dmerged), ctypes.c_int64(D), _p(merged),
       ctypes.c_int64(D), _p(ml), _p(cf_seq), ctypes.c_int64(S), _p(qkv_adj), ctypes.c_int64(3 * D), _p(cfh),
       _p(cf_seq_adj), ctypes.c_int64(S))
    return qkv_adj, cf_seq_adj, cfh


def linear(x, W, b=None, beta=0.0, out=None):
    """out = x W^T + b (+ beta out), fp64 accumulation."""
    lib = load()
    x, W = _c(x, np.float32), _c(W, np.float32)
    b = None if b is None else _c(b, np.float32)
    M, K = x.shape
    Nout = W.shape[0]
    out = np.zeros((M, Nout), dtype=np.float32) if out is None else _c(out, np.float32).copy()
    lib.oracle_linear_f32(_p(out), ctypes.c_int64(Nout), _p(x), ctypes.c_int64(K), _p(W), _p(b), M, Nout, K,
                          ctypes.c_float(beta))
    return out


def linear_bwd(g, W, beta=0.0, out=None):
    """in_adj = g W (+ beta in_adj), fp64 accumulation."""
    lib = load()
    g, W = _c(g, np.float32), _c(W, np.float32)
    M, Nout = g.shape
    K = W.shape[1]
    out = np.zeros((M, K), dtype=np.float32) if out is None else _c(out, np.float32).copy()
    lib.oracle_linear_bwd_f32(_p(out), ctypes.c_int64(K), _p(g), ctypes.c_int64(Nout), _p(W), M, Nout, K,
                              ctypes.c_float(beta))
    return out


def attention(qkv, off, cf_seq, w_out, b_out, heads, head_dim, temperature=1.0, N=None, dead=False):
    """(out, merged, ml) of the reference's attention()."""
    merged, ml = attn_fwd(qkv, off, cf_seq, heads, head_dim, temperature, N, dead)
    return linear(merged, w_out, b_out), merged, ml


def attention_bwd(out_adj, qkv, off, cf_seq, w_in, w_out, merged, ml, heads, head_dim, temperature=1.0,
                  cf_seq_adj=None, in_adj=None, beta=0.0, N=None, dead=False):
    """(in_adj, cf_seq_adj) of the reference's attention_bwd()."""
    dmerged = linear_bwd(out_adj, w_out)
    qkv_adj, cf_seq_adj, _ = attn_bwd(qkv, off, dmerged, merged, ml, cf_seq, heads, head_dim, temperature,
                                      cf_seq_adj, N, dead)
    return linear_bwd(qkv_adj, w_in, beta, in_adj), cf_seq_adj


# ---- the attention's input side and the consumer of its cf adjoint ---------

def cf_seq(off, cut, S):
    """cf_seq [N, S]: 1, then the atom's edges' cutoff factors, then 0
    (src/device_neighbors.cpp:318-323)."""
    lib = load()
    off = _c(off, np.int32)
    cut = _c(cut, np.float32)
    N = len(off) - 1
    out = np.zeros((N, S), dtype=np.float32)
    lib.oracle_cf_seq(N, S, _p(off), _p(cut), _p(out), ctypes.c_int64(S))
    return out


def norm_rows(x, w, b=None, dtype=np.float32):
    """RMSNorm (b None) or LayerNorm of each row (src/ops.hpp:376-407)."""
    lib = load()
    x, w = _c(x, dtype), _c(w, dtype)
    b = None if b is None else _c(b, dtype)
    rows, D = x.shape
    out = np.zeros_like(x)
    fn = lib.oracle_norm_rows_f32 if dtype == np.float32 else lib.oracle_norm_rows_f64
    fn(rows, D, _p(out), ctypes.c_int64(D), _p(x), ctypes.c_int64(D), _p(w), _p(b))
    return out


def norm_rows_bwd(g, x, w, ln, beta=0.0, in_adj=None, dtype=np.float32):
    """beta in_adj + the norm's input adjoint for output adjoint g (src/ops.hpp:409-436)."""
    lib = load()
    g, x, w = _c(g, dtype), _c(x, dtype), _c(w, dtype)
    rows, D = x.shape
    out = np.zeros_like(x) if in_adj is None else _c(in_adj, dtype).copy()
    if dtype == np.float32:
        lib.oracle_norm_rows_bwd_f32(rows, D, _p(out), ctypes.c_int64(D), ctypes.c_float(beta), _p(g),
                                     ctypes.c_int64(D), _p(x), ctypes.c_int64(D), _p(w), int(ln))
    else:
        lib.oracle_norm_rows_bwd_f64(rows, D, _p(out), ctypes.c_int64(D), ctypes.c_double(beta), _p(g),
                                     ctypes.c_int64(D), _p(x), ctypes.c_int64(D), _p(w), int(ln))
    return out


def cutoff(d, rc, width, kind, f64=False):
    """(value, d value / d dist) of the smooth cutoff `kind` (0 bump, 1 cosine,
    2 smooth), transcendentals in float as the reference's CutT unless f64
    (include/pet/cutoff.hpp:17-35, src/forces.cpp:21-42)."""
    lib = load()
    d = _c(np.atleast_1d(d), np.float64)
    rc = _c(np.broadcast_to(rc, d.shape), np.float64)
    v, dd = np.zeros_like(d), np.zeros_like(d)
    lib.oracle_cutoff(len(d), _p(d), _p(rc), ctypes.c_double(width), int(kind), int(f64), _p(v), _p(dd))
    return v, dd


def edge_grad(off, center, x4_adj, cutoff_adj, cf_seq_adj, vec, dist, pcut, width, kind, n_edges=None):
    """grad [E, 3] fp64 of forces_and_virial's edge pass (src/forces.cpp:364-378)."""
    lib = load()
    off, center = _c(off, np.int32), _c(center, np.int32)
    x4_adj = _c(x4_adj, np.float32)
    cutoff_adj = None if cutoff_adj is None else _c(cutoff_adj, np.float32)
    cf_seq_adj = _c(cf_seq_adj, np.float32)
    vec, dist, pcut = _c(vec, np.float64), _c(dist, np.float64), _c(pcut, np.float64)
    E = len(center) if n_edges is None else n_edges
    grad = np.zeros((E, 3), dtype=np.float64)
    lib.oracle_edge_grad(len(off) - 1, E, _p(off), _p(center), _p(x4_adj), ctypes.c_int64(4), _p(cutoff_adj),
                         _p(cf_seq_adj), ctypes.c_int64(cf_seq_adj.shape[1]), _p(vec), _p(dist), _p(pcut),
                         ctypes.c_double(width), int(kind), _p(grad))
    return grad


def fold(N, off, rev, vec, grad, scale=1.0):
    """(forces [N, 3], per-atom virial [N, 9]) of fold_edge_gradients (src/forces.cpp:50-68)."""
    lib = load()
    off, rev = _c(off, np.int32), _c(rev, np.int32)
    vec, grad = _c(vec, np.float64), _c(grad, np.float64)
    forces = np.zeros((N, 3), dtype=np.float64)
    vir = np.zeros((N, 9), dtype=np.float64)
    lib.oracle_fold(N, len(off) - 1, _p(off), _p(rev), _p(vec), _p(grad), ctypes.c_double(scale), _p(forces),
                    _p(vir))
    return forces, vir


def struct_sum(soff, x, out=None, acc=False):
    """Per-structure sums of x's rows (src/forces.cpp:287-302)."""
    lib = load()
    soff = _c(soff, np.int32)
    x = _c(x, np.float64)
    NS, W = len(soff) - 1, x.shape[1]
    out = np.zeros((NS, W), dtype=np.float64) if out is None else _c(out, np.float64).copy()
    lib.oracle_struct_sum(NS, W, _p(soff), _p(x), _p(out), int(acc))
    return out
