"""Seeded structures, neighbour lists and the attention's token layout.

The workloads of the benchmark configurations, built the way the reference
builds its inputs:

- raw edges in the order of ``build_raw_edges`` (reference
  src/neighbors.cpp:68-97): for each centre i, for each atom j, for each
  periodic image (sa, sb, sc) in lexicographic order, every pair within the
  cutoff except an atom with itself;
- kept edges (every raw edge when the cutoff is not adaptive) fill an atom's
  slots in that order (src/neighbors.cpp:176-247);
- the cosine cutoff factor 0.5 (1 + cos(pi x)), x = clamp((d - (rc - w)) / w,
  0, 1) (src/neighbors.cpp:38-41);
- ``cf_seq[n, 0] = 1`` (the central token), ``cf_seq[n, 1 + m]`` = slot m's
  factor, 0 past the atom's edges (src/model.cpp:375-377), stored as fp32;
- ``off`` = the exclusive prefix sum of per-atom kept edges (the CSR of
  ``pack_edges``, src/model.cpp:531-537); atom n's tokens are row n and rows
  N + off[n] .. N + off[n+1] - 1 (src/ops.hpp:31-37).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

DIAMOND_A = 3.567  # Angstrom


@dataclasses.dataclass
class Structure:
    positions: np.ndarray  # [N, 3] float64
    cell: np.ndarray  # [3, 3] float64, rows are lattice vectors
    numbers: np.ndarray  # [N] int
    pbc: tuple = (True, True, True)


def diamond(ncell: int, a: float = DIAMOND_A, jitter: float = 0.0, seed: int = 0) -> Structure:
    """ncell^3 conventional cubic cells of diamond (8 atoms each), each
    position displaced by N(0, jitter) (Angstrom) from ``seed``."""
    fcc = np.array([[0, 0, 0], [0, 0.5, 0.5], [0.5, 0, 0.5], [0.5, 0.5, 0]], dtype=np.float64)
    basis = np.concatenate([fcc, fcc + 0.25])
    cells = np.array([[i, j, k] for i in range(ncell) for j in range(ncell) for k in range(ncell)], dtype=np.float64)
    frac = (cells[:, None, :] + basis[None, :, :]).reshape(-1, 3)
    pos = frac * a
    if jitter > 0:
        pos = pos + np.random.default_rng(seed).normal(0.0, jitter, size=pos.shape)
    L = ncell * a
    return Structure(pos, np.eye(3) * L, np.full(len(pos), 6, dtype=np.int64))


def water_box(n_side: int = 6, box: float = 18.6, seed: int = 0, r_oh: float = 0.96,
              angle_deg: float = 104.5) -> Structure:
    """n_side^3 water molecules (216 by default: 1.0 g/cm^3 in an 18.6 A cube)
    with their oxygens on a cubic grid and uniformly random orientations."""
    rng = np.random.default_rng(seed)
    spacing = box / n_side
    half = math.radians(angle_deg) / 2
    local = np.array([[0.0, 0.0, 0.0],
                      [r_oh * math.sin(half), 0.0, r_oh * math.cos(half)],
                      [-r_oh * math.sin(half), 0.0, r_oh * math.cos(half)]])
    pos, numbers = [], []
    for i in range(n_side):
        for j in range(n_side):
            for k in range(n_side):
                o = (np.array([i, j, k], dtype=np.float64) + 0.5) * spacing
                q = rng.normal(size=4)
                q /= np.linalg.norm(q)
                w, x, y, z = q
                rot = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                                [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                                [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])
                pos.append(o + local @ rot.T)
                numbers += [8, 1, 1]
    return Structure(np.concatenate(pos), np.eye(3) * box, np.array(numbers, dtype=np.int64))


def random_box(n_atoms: int = 4096, density: float = 0.1, seed: int = 0) -> Structure:
    """n_atoms uniformly at random in a periodic cube of the given number
    density (atoms per A^3)."""
    L = (n_atoms / density) ** (1.0 / 3.0)
    pos = np.random.default_rng(seed).uniform(0.0, L, size=(n_atoms, 3))
    return Structure(pos, np.eye(3) * L, np.full(n_atoms, 6, dtype=np.int64))


def image_ranges(cell: np.ndarray, cutoff: float, pbc=(True, True, True)):
    """Images per direction: the cutoff over the interplanar spacing, rounded
    up (src/neighbors.cpp:53-66)."""
    a, b, c = cell
    vol = abs(np.dot(a, np.cross(b, c)))
    if vol < 1e-12:
        return (0, 0, 0)
    faces = [np.cross(b, c), np.cross(c, a), np.cross(a, b)]
    return tuple(int(math.ceil(cutoff / (vol / np.linalg.norm(f)))) if p else 0 for f, p in zip(faces, pbc))


@dataclasses.dataclass
class Edges:
    centre: np.ndarray  # [E] int32
    neigh: np.ndarray  # [E] int32
    vec: np.ndarray  # [E, 3] float64, r_j + shift - r_i
    dist: np.ndarray  # [E] float64
    shift: np.ndarray | None = None  # [E, 3] int, the image of r_j in cell units


def neighbor_list(s: Structure, cutoff: float) -> Edges:
    """Every ordered pair (i, j, image) with 0 < |v| <= cutoff, in the raw-edge
    order of the reference's build_raw_edges."""
    rng = image_ranges(s.cell, cutoff, s.pbc)
    shifts = np.array([[sa, sb, sc] for sa in range(-rng[0], rng[0] + 1)
                       for sb in range(-rng[1], rng[1] + 1) for sc in range(-rng[2], rng[2] + 1)], dtype=np.float64)
    svec = shifts @ s.cell  # [I, 3]
    x = s.positions
    N = len(x)
    c2 = cutoff * cutoff
    cen, nei, vecs, dists, shs = [], [], [], [], []
    # images of every atom: [N, I, 3], flattened j-major then image, the reference's loop order
    img = (x[:, None, :] + svec[None, :, :]).reshape(-1, 3)
    jj = np.repeat(np.arange(N, dtype=np.int32), len(svec))
    ss = np.tile(shifts.astype(np.int64), (N, 1))
    for i in range(N):
        v = img - x[i]
        d2 = np.einsum("ij,ij->i", v, v)
        keep = (d2 >= 1e-24) & (d2 <= c2)
        idx = np.nonzero(keep)[0]
        cen.append(np.full(len(idx), i, dtype=np.int32))
        nei.append(jj[idx])
        vecs.append(v[idx])
        dists.append(np.sqrt(d2[idx]))
        shs.append(ss[idx])
    return Edges(np.concatenate(cen), np.concatenate(nei), np.concatenate(vecs), np.concatenate(dists),
                 np.concatenate(shs))


def cosine_cutoff(d: np.ndarray, rc: float, width: float) -> np.ndarray:
    x = np.clip((d - (rc - width)) / width, 0.0, 1.0)
    return 0.5 * (1.0 + np.cos(np.pi * x))


@dataclasses.dataclass
class PackedEdges:
    """An atom's kept edges contiguous (CSR ``off``), as the reference's
    PackedEdges (include/pet/model.hpp:153-168): each edge's centre, its
    reverse (j, i, -shift) edge or -1, vector, length, pair cutoff and smooth
    cutoff factor."""
    off: np.ndarray  # [N+1] int32
    center: np.ndarray  # [E] int32
    neigh: np.ndarray  # [E] int32
    reverse: np.ndarray  # [E] int32
    vec: np.ndarray  # [E, 3] float64
    dist: np.ndarray  # [E] float64
    pcut: np.ndarray  # [E] float64
    cut: np.ndarray  # [E] float32


def packed_edges(n_atoms: int, e: Edges, cutoff: float, width: float = 0.5) -> PackedEdges:
    """The full directed edge list in the raw order (already grouped by centre),
    with reverse indices from the image shifts and cosine cutoff factors."""
    E = len(e.centre)
    counts = np.bincount(e.centre, minlength=n_atoms)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    assert np.all(np.diff(e.centre) >= 0), "edges must be grouped by centre"
    index = {(int(i), int(j), *map(int, sh)): k for k, (i, j, sh) in enumerate(zip(e.centre, e.neigh, e.shift))}
    rev = np.array([index.get((int(j), int(i), *map(int, -sh)), -1) for i, j, sh in zip(e.centre, e.neigh, e.shift)],
                   dtype=np.int32) if E else np.zeros(0, dtype=np.int32)
    cut = cosine_cutoff(e.dist, cutoff, width).astype(np.float32)
    return PackedEdges(off, e.centre.astype(np.int32), e.neigh.astype(np.int32), rev, e.vec.astype(np.float64),
                       e.dist.astype(np.float64), np.full(E, cutoff, dtype=np.float64), cut)


@dataclasses.dataclass
class Tokens:
    """The attention's token layout: CSR offsets and cutoff factors."""
    off: np.ndarray  # [N+1] int32
    cf_seq: np.ndarray  # [N, S] float32
    n_atoms: int
    n_edges: int
    slots: int

    @property
    def n_rows(self) -> int:
        return self.n_atoms + self.n_edges

    def counts(self) -> np.ndarray:
        return np.diff(self.off) + 1

    def rows(self, n: int) -> np.ndarray:
        """Token rows of atom n in slot order."""
        return np.concatenate([[n], self.n_atoms + np.arange(self.off[n], self.off[n + 1])]).astype(np.int64)


def tokens_from_edges(n_atoms: int, edges: Edges, cutoff: float, width: float = 0.5,
                      slots: int | None = None) -> Tokens:
    counts = np.bincount(edges.centre, minlength=n_atoms)
    off = np.zeros(n_atoms + 1, dtype=np.int64)
    off[1:] = np.cumsum(counts)
    M = max(1, int(counts.max()) if n_atoms else 0)
    S = M + 1 if slots is None else slots
    if S < M + 1:
        raise ValueError(f"slots {S} below the largest count {M + 1}")
    cf = np.zeros((n_atoms, S), dtype=np.float64)
    cf[:, 0] = 1.0
    fac = cosine_cutoff(edges.dist, cutoff, width)
    slot = np.arange(len(edges.centre)) - off[edges.centre]
    cf[edges.centre, 1 + slot] = fac
    return Tokens(off.astype(np.int32), cf.astype(np.float32), n_atoms, int(off[-1]), S)


def tokens_from_counts(counts, seed: int = 0, slots: int | None = None, cf_kind: str = "random") -> Tokens:
    """A synthetic layout from per-atom edge counts, cutoff factors drawn in
    (0, 1] ("random"), all one ("ones"), or random with some exact zeros
    ("zeros": edges at their cutoff)."""
    counts = np.asarray(counts, dtype=np.int64)
    N = len(counts)
    rng = np.random.default_rng(seed)
    off = np.zeros(N + 1, dtype=np.int64)
    off[1:] = np.cumsum(counts)
    S = int(counts.max()) + 1 if slots is None else slots
    cf = np.zeros((N, S), dtype=np.float64)
    cf[:, 0] = 1.0
    for n, m in enumerate(counts):
        if cf_kind == "ones":
            v = np.ones(m)
        else:
            v = rng.uniform(0.05, 1.0, size=m)
            if cf_kind == "zeros" and m > 0:
                v[rng.random(m) < 0.25] = 0.0
        cf[n, 1:1 + m] = v
    return Tokens(off.astype(np.int32), cf.astype(np.float32), N, int(off[-1]), S)


# ---- the benchmark configurations ------------------------------------------------

@dataclasses.dataclass
class AttnConfig:
    name: str
    structure: str
    d_model: int
    heads: int
    cutoff: float
    width: float = 0.5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.heads


CONFIGS = {
    # the CPU-runnable attention op
    "c1": AttnConfig("diamond-64", "diamond:2:0.01", 128, 4, 4.5),
    # the north-star attention workload
    "c3": AttnConfig("diamond-1728", "diamond:6:0.02", 256, 8, 4.5),
    # ragged segments
    "c4": AttnConfig("ragged-4096", "random:4096:0.1", 256, 8, 5.0),
    # configs[1] geometry at the attention shapes of its model (d 128, 4 heads)
    "c2": AttnConfig("water-648", "water:6:18.6", 128, 4, 4.5),
    # 32 structures in one call, alternating diamond-64 and water-648
    "c5": AttnConfig("batch-32", "batch:16", 512, 8, 4.5),
}


def batch_edges(n_pairs: int = 16, cutoff: float = 4.5, seed: int = 0):
    """2 n_pairs independent structures (diamond-64 and water-648 alternating,
    each seeded by its index) as one atom list: (atoms, edges with atom
    indices offset per structure, per-structure atom offsets soff)."""
    parts, soff, base = [], [0], 0
    for k in range(2 * n_pairs):
        st = diamond(2, jitter=0.01, seed=seed + k) if k % 2 == 0 else water_box(6, 18.6, seed=seed + k)
        e = neighbor_list(st, cutoff)
        parts.append(Edges(e.centre + base, e.neigh + base, e.vec, e.dist, e.shift))
        base += len(st.positions)
        soff.append(base)
    cat = lambda f: np.concatenate([getattr(p, f) for p in parts])
    return base, Edges(cat("centre").astype(np.int32), cat("neigh").astype(np.int32), cat("vec"), cat("dist"),
                       cat("shift")), np.array(soff, dtype=np.int32)


def build_structure(spec: str, seed: int = 0) -> Structure:
    kind, *args = spec.split(":")
    if kind == "diamond":
        return diamond(int(args[0]), jitter=float(args[1]), seed=seed)
    if kind == "random":
        return random_box(int(args[0]), float(args[1]), seed=seed)
    if kind == "water":
        return water_box(int(args[0]), float(args[1]), seed=seed)
    raise ValueError(spec)


def config_tokens(name: str, seed: int = 0) -> tuple[AttnConfig, Tokens]:
    cfg = CONFIGS[name]
    if cfg.structure.startswith("batch:"):
        N, e, _ = batch_edges(int(cfg.structure.split(":")[1]), cfg.cutoff, seed)
        return cfg, tokens_from_edges(N, e, cfg.cutoff, cfg.width)
    s = build_structure(cfg.structure, seed)
    e = neighbor_list(s, cfg.cutoff)
    return cfg, tokens_from_edges(len(s.positions), e, cfg.cutoff, cfg.width)


def attention_inputs(tk: Tokens, d_model: int, heads: int, seed: int = 0, dtype=np.float32):
    """Random-init weights and activations of one attention layer: token
    features N(0, 1), W_in [3D, D] and W_out [D, D] with entries N(0, 1/sqrt(D)),
    small biases, qkv = tokens W_in^T + b_in, and an output adjoint N(0, 1)."""
    rng = np.random.default_rng(seed)
    D, T = d_model, tk.n_rows
    x = rng.standard_normal((T, D)).astype(np.float32)
    w_in = (rng.standard_normal((3 * D, D)) / math.sqrt(D)).astype(np.float32)
    b_in = (0.1 * rng.standard_normal(3 * D)).astype(np.float32)
    w_out = (rng.standard_normal((D, D)) / math.sqrt(D)).astype(np.float32)
    b_out = (0.1 * rng.standard_normal(D)).astype(np.float32)
    qkv = (x.astype(np.float64) @ w_in.T.astype(np.float64) + b_in).astype(np.float32)
    out_adj = rng.standard_normal((T, D)).astype(np.float32)
    return dict(x=x.astype(dtype), w_in=w_in.astype(dtype), b_in=b_in.astype(dtype), w_out=w_out.astype(dtype),
                b_out=b_out.astype(dtype), qkv=qkv.astype(dtype), out_adj=out_adj.astype(dtype))
