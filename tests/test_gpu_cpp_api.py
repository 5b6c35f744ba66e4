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
