"""The C++ interface (include/pet/attention.hpp: pet::attention,
pet::attention_bwd, pet::Workspace) driven by a compiled C++ caller
(tests/cpp/attention_api_test.cpp) and checked against the oracle."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import oracle
from pet_kokkos_amd import build as B
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def rel(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / np.abs(b).max())


@pytest.mark.parametrize("beta,temperature", [(0.0, 1.0), (1.0, 0.7)])
def test_cpp_attention_api(tmp_path, beta, temperature):
    if not os.path.exists(B.CPP_TEST):
        pytest.fail(f"{B.CPP_TEST} is not built (python -m pet_kokkos_amd.build)")
    conf, tk = systems.config_tokens("c2")
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    inp = systems.attention_inputs(tk, D, H, seed=3)
    rng = np.random.default_rng(11)
    in_adj0 = rng.standard_normal((tk.n_rows, D)).astype(np.float32)
    cf_adj0 = rng.standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)
    files = dict(qkv=inp["qkv"], cf=tk.cf_seq, w_in=inp["w_in"], w_out=inp["w_out"], b_out=inp["b_out"],
                 out_adj=inp["out_adj"], in_adj0=in_adj0, cf_adj0=cf_adj0)
    for k, v in files.items():
        np.ascontiguousarray(v, dtype=np.float32).tofile(tmp_path / f"{k}.f32")
    np.ascontiguousarray(tk.off, dtype=np.int32).tofile(tmp_path / "off.i32")
    args = [B.CPP_TEST, str(tmp_path), tk.n_atoms, tk.n_rows, tk.slots, H, hd, temperature, beta, D]
    print(f"[gpu] C++ API water-648 beta={beta}", flush=True)
    res = subprocess.run([str(a) for a in args], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    out = np.fromfile(tmp_path / "out.f32", dtype=np.float32).reshape(tk.n_rows, D)
    in_adj = np.fromfile(tmp_path / "in_adj.f32", dtype=np.float32).reshape(tk.n_rows, D)
    cf_adj = np.fromfile(tmp_path / "cf_adj.f32", dtype=np.float32).reshape(tk.n_atoms, tk.slots)
    rout, rm, rml = oracle.attention(inp["qkv"], tk.off, tk.cf_seq, inp["w_out"], inp["b_out"], H, hd, temperature)
    rin, rca = oracle.attention_bwd(inp["out_adj"], inp["qkv"], tk.off, tk.cf_seq, inp["w_in"], inp["w_out"], rm, rml,
                                    H, hd, temperature, cf_seq_adj=cf_adj0, in_adj=in_adj0, beta=beta)
    assert rel(out, rout) <= RTOL
    assert rel(in_adj, rin) <= RTOL
    assert rel(cf_adj, rca) <= RTOL
    assert (tmp_path / "repeat.ok").exists(), "a warm workspace's second backward differed"


def test_cpp_layer_and_forces_api(tmp_path):
    """cf_seq, attention_layer, attention_layer_bwd and forces_and_virial
    (include/pet/attention.hpp, include/pet/forces.hpp) from a compiled C++
    caller on the C1 geometry, against the oracle's chain of the same steps."""
    if not os.path.exists(B.CPP_TEST2):
        pytest.fail(f"{B.CPP_TEST2} is not built (python -m pet_kokkos_amd.build)")
    cfg = systems.CONFIGS["c1"]
    s = systems.build_structure(cfg.structure, 0)
    e = systems.neighbor_list(s, cfg.cutoff)
    N = len(s.positions)
    pk = systems.packed_edges(N, e, cfg.cutoff, cfg.width)
    tk = systems.tokens_from_edges(N, e, cfg.cutoff, cfg.width)
    H, hd, D, E, S, T = cfg.heads, cfg.head_dim, cfg.d_model, len(pk.center), tk.slots, tk.n_rows
    inp = systems.attention_inputs(tk, D, H, seed=8)
    rng = np.random.default_rng(9)
    tokens = rng.standard_normal((T, D)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    x4 = rng.standard_normal((E, 4)).astype(np.float32)
    f32 = dict(tokens=tokens, nw=nw, w_in=inp["w_in"], b_in=inp["b_in"], w_out=inp["w_out"], b_out=inp["b_out"],
               cut=pk.cut, out_adj=inp["out_adj"], x4=x4)
    for k, v in f32.items():
        np.ascontiguousarray(v, dtype=np.float32).tofile(tmp_path / f"{k}.f32")
    for k, v in dict(off=pk.off, center=pk.center, reverse=pk.reverse).items():
        np.ascontiguousarray(v, dtype=np.int32).tofile(tmp_path / f"{k}.i32")
    for k, v in dict(vec=pk.vec, dist=pk.dist, pcut=pk.pcut).items():
        np.ascontiguousarray(v, dtype=np.float64).tofile(tmp_path / f"{k}.f64")
    print("[gpu] C++ layer + forces API diamond-64", flush=True)
    res = subprocess.run([str(a) for a in (B.CPP_TEST2, tmp_path, N, T, S, H, hd, E)], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    rd = lambda k, dt, shp: np.fromfile(tmp_path / k, dtype=dt).reshape(shp)
    rcf = oracle.cf_seq(pk.off, pk.cut, S)
    assert np.array_equal(rd("cf.f32", np.float32, (N, S)), rcf)
    qkv = oracle.linear(oracle.norm_rows(tokens, nw, None), inp["w_in"], inp["b_in"])
    rout, rm, rml = oracle.attention(qkv, pk.off, rcf, inp["w_out"], inp["b_out"], H, hd, 1.0)
    assert rel(rd("out.f32", np.float32, (T, D)), rout) <= RTOL
    n_adj, rcsa = oracle.attention_bwd(inp["out_adj"], qkv, pk.off, rcf, inp["w_in"], inp["w_out"], rm, rml, H, hd, 1.0)
    rtadj = oracle.norm_rows_bwd(n_adj, tokens, nw, False)
    assert rel(rd("tokens_adj.f32", np.float32, (T, D)), rtadj) <= RTOL
    assert rel(rd("cf_adj.f32", np.float32, (N, S)), rcsa) <= RTOL
    rg = oracle.edge_grad(pk.off, pk.center, x4, None, rcsa, pk.vec, pk.dist, pk.pcut, 0.5, 1)
    assert rel(rd("grad.f64", np.float64, (E, 3)), rg) <= RTOL
    rf, rv = oracle.fold(N, pk.off, pk.reverse, pk.vec, rg, scale=-1.0)
    assert rel(rd("forces.f64", np.float64, (N, 3)), rf) <= RTOL
    assert rel(rd("vir9.f64", np.float64, (9,)), rv.sum(axis=0)) <= RTOL
    assert (tmp_path / "graph.ok").exists(), "pet::StepRecorder: a recorded or replayed run differed from the eager one"


@pytest.mark.parametrize("name", ["tiny", "tiny-residual"])
def test_cpp_model_calculator(tmp_path, name):
    """pet::PetModel + pet::Calculator (include/pet/model.hpp) from C++: the
    C++ host neighbour list, the model's energy / forces / virial against the
    CPU oracle, a repeat bit for bit, and forces against a central difference
    of the energy, and compute_step replayed as a HIP graph giving the bits of
    eager steps."""
    from oracle import pet_model as om
    from pet_kokkos_amd import weights
    from pet_kokkos_amd.forces import CUTOFF_KINDS
    from pet_kokkos_amd.model import species_index

    if not os.path.exists(B.CPP_TEST3):
        pytest.fail(f"{B.CPP_TEST3} is not built (python -m pet_kokkos_amd.build)")
    h = weights.MODELS[name]
    w = weights.random_weights(h, 21)
    comp = weights.random_composition(h)
    s = systems.water_box(2, 6.2, seed=8)
    N = len(s.positions)
    with open(tmp_path / "hypers.txt", "w") as f:
        f.write(f"{h.d_pet} {h.d_node} {h.d_head} {h.num_heads} {h.num_gnn_layers} {h.num_attention_layers} "
                f"{h.n_species} {CUTOFF_KINDS[h.cutoff_function]} {h.cutoff_width} {h.attention_temperature} 1.0 "
                f"{h.cutoff} {1 if h.residual else 0}\n")
    with open(tmp_path / "manifest.txt", "w") as f, open(tmp_path / "weights.f64", "wb") as g:
        for k, v in w.items():
            f.write(f"{k} {v.shape[0]} {v.shape[1] if v.ndim == 2 else 0}\n")
            np.ascontiguousarray(v, dtype=np.float64).tofile(g)
    np.ascontiguousarray(comp, dtype=np.float64).tofile(tmp_path / "composition.f64")
    s2i = [-1] * (max(h.atomic_types) + 1)
    for i, z in enumerate(h.atomic_types):
        s2i[z] = i
    (tmp_path / "s2i.txt").write_text(" ".join(map(str, s2i)))
    with open(tmp_path / "system.txt", "w") as f:
        f.write(f"{N}\n" + " ".join(f"{c:.17g}" for c in s.cell.reshape(-1)) + "\n")
        for z, p in zip(s.numbers, s.positions):
            f.write(f"{int(z)} {p[0]:.17g} {p[1]:.17g} {p[2]:.17g}\n")
    print("[gpu] C++ model water-24", flush=True)
    res = subprocess.run([B.CPP_TEST3, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    r = np.fromfile(tmp_path / "result.f64", dtype=np.float64)
    energy, pa, forces, vir = r[0], r[1:1 + N], r[1 + N:1 + 4 * N].reshape(N, 3), r[1 + 4 * N:].reshape(3, 3)
    pk = systems.packed_edges(N, systems.neighbor_list(s, h.cutoff), h.cutoff, h.cutoff_width)
    rpa, eg = om.evaluate(h, w, species_index(s.numbers, h.atomic_types), pk, comp)
    rf, rvir = om.fold_forces(N, pk, eg)
    assert abs(energy - rpa.sum()) <= 1e-6 * abs(rpa.sum())
    assert np.abs(pa - rpa).max() <= 1e-5 * np.abs(rpa).max()
    assert np.abs(forces - rf).max() <= 1e-5 * np.abs(rf).max()
    assert np.abs(vir - rvir.sum(0).reshape(3, 3)).max() <= 1e-5 * np.abs(rvir).sum(0).max()
    assert os.path.exists(tmp_path / "repeat.ok")
    fd, f0 = np.fromfile(tmp_path / "fd.f64", dtype=np.float64)
    assert abs(fd - f0) <= 1e-2 + 1e-3 * abs(f0), (fd, f0)
    assert (tmp_path / "graph.ok").exists(), "Calculator(graph = true): a replayed step differed from an eager one"
    assert (tmp_path / "linear.ok").exists(), "pet::linear_fused (plain or split weights) missed the host product"
    assert (tmp_path / "pairs.ok").exists(), "pet::dense_pairs missed the bits of pet::dense on split weights"
