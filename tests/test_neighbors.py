"""The host neighbour lists -- Python systems.neighbor_list (which feeds the
oracle and the product alike in every model test) and C++ pet::build_edges
(include/pet/model.hpp, the Calculator's) -- against an independent brute
force, without a GPU.

The reference's raw edges (src/neighbors.cpp:76-97, kept edges in that order
by :176-247): for each centre i, for each atom j, for each periodic image
(sa, sb, sc) in lexicographic order, every pair with 1e-24 <= d^2 <= rc^2.
The brute force here does not use the interplanar image count: it walks a
fixed generous image range with scalar arithmetic (small systems), or, for
larger ones, finds each pair's minimum image from fractional coordinates and
enumerates images around it. Diamond fixes a count: 70 neighbours an atom at
4.5 A (shells at 1.545, 2.522, 2.958, 3.567, 3.887, 4.369 A of 4, 12, 12, 6,
12 and 24 atoms; the next at 4.634 A).
"""
from __future__ import annotations

import itertools
import math
import os
import subprocess

import numpy as np
import pytest

from pet_kokkos_amd import systems

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def brute_force_scalar(s, rc, extra=1):
    """(i, j, sa, sb, sc) in the reference's order, scalar arithmetic over a
    fixed image range wide enough for any cell whose shortest height exceeds
    rc / (reach - extra)."""
    heights = [abs(np.linalg.det(s.cell)) / np.linalg.norm(np.cross(s.cell[(k + 1) % 3], s.cell[(k + 2) % 3]))
               for k in range(3)]
    reach = [int(math.ceil(rc / h)) + extra for h in heights]
    out = []
    x = s.positions.tolist()
    cell = s.cell.tolist()
    for i in range(len(x)):
        for j in range(len(x)):
            for sa in range(-reach[0], reach[0] + 1):
                for sb in range(-reach[1], reach[1] + 1):
                    for sc in range(-reach[2], reach[2] + 1):
                        v = [x[j][c] + sa * cell[0][c] + sb * cell[1][c] + sc * cell[2][c] - x[i][c] for c in range(3)]
                        d2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2]
                        if 1e-24 <= d2 <= rc * rc:
                            out.append((i, j, sa, sb, sc))
    return out


def brute_force_minimum_image(s, rc):
    """The same set by another route: each pair's minimum image from wrapped
    fractional displacements, then every image within the reach of it."""
    inv = np.linalg.inv(s.cell)
    frac = s.positions @ inv
    heights = [abs(np.linalg.det(s.cell)) / np.linalg.norm(np.cross(s.cell[(k + 1) % 3], s.cell[(k + 2) % 3]))
               for k in range(3)]
    reach = [int(math.ceil(rc / h)) + 1 for h in heights]
    around = np.array(list(itertools.product(*[range(-r, r + 1) for r in reach])))
    out = set()
    for i in range(len(frac)):
        df = frac - frac[i]
        base = -np.round(df)  # minimum image shift per j
        for j in range(len(frac)):
            sh = base[j][None, :] + around  # [I, 3]
            v = (df[j][None, :] + sh) @ s.cell
            d2 = (v * v).sum(1)
            for k in np.nonzero((d2 >= 1e-24) & (d2 <= rc * rc))[0]:
                out.add((i, j, *map(int, sh[k])))
    return out


def listed(e):
    return [(int(i), int(j), *map(int, t)) for i, j, t in zip(e.centre, e.neigh, e.shift)]


def test_diamond_64_order_and_count():
    s = systems.diamond(2, jitter=0.01, seed=0)
    e = systems.neighbor_list(s, 4.5)
    got = listed(e)
    assert got == brute_force_scalar(s, 4.5)
    assert np.all(np.bincount(e.centre, minlength=64) == 70)
    # the shells of perfect diamond
    d = np.sort(np.unique(np.round(systems.neighbor_list(systems.diamond(2), 4.5).dist, 3)))
    assert np.allclose(d, [1.545, 2.522, 2.958, 3.567, 3.887, 4.369], atol=1e-3)
    # vectors and distances are those of the listed images
    v = s.positions[e.neigh] + e.shift @ s.cell - s.positions[e.centre]
    assert np.abs(v - e.vec).max() < 1e-12 and np.abs(np.linalg.norm(v, axis=1) - e.dist).max() < 1e-12


@pytest.mark.parametrize("case", ["water-648", "ragged-512", "triclinic"])
def test_larger_systems_as_sets(case):
    if case == "water-648":
        s, rc = systems.water_box(6, 18.6, seed=0), 4.5
    elif case == "ragged-512":
        s, rc = systems.random_box(512, 0.1, seed=1), 5.0
    else:  # a sheared cell, so the image range is not the same along each vector
        s = systems.diamond(2, jitter=0.02, seed=3)
        s.cell = np.array([[7.134, 0.0, 0.0], [2.5, 7.134, 0.0], [1.0, -1.5, 7.134]])
        rc = 4.5
    e = systems.neighbor_list(s, rc)
    got = listed(e)
    ref = brute_force_minimum_image(s, rc)
    assert len(got) == len(set(got)) and set(got) == ref
    # reference order: centre-major, then j, then the image lexicographically
    assert got == sorted(got)
    counts = np.bincount(e.centre, minlength=len(s.positions))
    if case == "water-648":
        assert 30 <= counts.mean() <= 45  # about 38 at 1 g/cm^3 and 4.5 A
    if case == "ragged-512":
        assert counts.min() < counts.max()  # ragged


def test_cpp_build_edges(tmp_path):
    exe = tmp_path / "neighbors_dump"
    cmd = ["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-o", str(exe),
           os.path.join(ROOT, "tests", "cpp", "neighbors_dump.cpp")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.fail(res.stderr)
    for s, rc in ((systems.diamond(2, jitter=0.01, seed=0), 4.5), (systems.water_box(3, 9.3, seed=2), 4.5)):
        inp = tmp_path / "s.txt"
        with open(inp, "w") as f:
            f.write(f"{len(s.positions)}\n")
            for r in s.cell:
                f.write(" ".join(repr(float(v)) for v in r) + "\n")
            for p in s.positions:
                f.write(" ".join(repr(float(v)) for v in p) + "\n")
        out = tmp_path / "e.txt"
        res = subprocess.run([str(exe), str(inp), str(out), repr(rc)], capture_output=True, text=True)
        assert res.returncode == 0, res.stderr
        rows = np.loadtxt(out, dtype=np.int64).reshape(-1, 6)
        got = [tuple(map(int, r[:5])) for r in rows]
        assert got == listed(systems.neighbor_list(s, rc))
        assert set(got) == brute_force_minimum_image(s, rc)
        # each edge's reverse is (j, i, -shift)
        for k, (i, j, a, b, c, rv) in enumerate(rows):
            assert rv >= 0 and tuple(rows[rv][:5]) == (j, i, -a, -b, -c)
