"""The chunked forms (reference attention_chunked / attention_bwd_chunked,
src/attention.cpp:2055-2187, and its test of PET_EDGE_CHUNK=37 giving the same
bits, tests/test_determinism.cpp:207-236), on an MI355X.

Run-level kernels over runs of atoms must give the same bits as the whole-
matrix call: every item's arithmetic is the same. The op level adds the
W_out / W_in GEMMs per run (rocBLAS, whose kernel choice can depend on the
number of rows), so it is held to the parity tolerance and its bitwise
agreement is reported.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from parity import row_err
from pet_kokkos_amd import _lib
from pet_kokkos_amd import attention as A
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu
RTOL = 1e-5


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def run_rows(N, n0, n1, e0, e1):
    return torch.cat([torch.arange(n0, n1), torch.arange(N + e0, N + e1)])


@pytest.mark.parametrize("cfg,chunk,stream", [("c1", 37, 0), ("c1", 300, 0), ("c2", 500, 0), ("c4", 4000, 0),
                                              ("c1", 37, 1), ("c4", 4000, 1)])
def test_runs_bit_identical(device, cfg, chunk, stream):
    with _lib.options(attn_stream=stream):
        _runs_bit_identical(device, cfg, chunk, stream)


def _runs_bit_identical(device, cfg, chunk, stream):
    conf, tk = systems.config_tokens(cfg)
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    print(f"[gpu] runs {cfg} chunk {chunk} streaming kernels {stream}", flush=True)
    inp = systems.attention_inputs(tk, D, H, seed=4)
    rng = np.random.default_rng(5)
    q = torch.from_numpy(inp["qkv"]).to(device)
    dm = torch.from_numpy(rng.standard_normal((tk.n_rows, D)).astype(np.float32)).to(device)
    off = torch.from_numpy(tk.off).to(device)
    cf = torch.from_numpy(tk.cf_seq).to(device)
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    merged, ml = A.attn_fwd(q, off, cf, H, hd)
    qa, ca, cfh = A.attn_bwd(q, off, dm, merged, ml, cf, H, hd)
    merged2 = torch.zeros_like(merged)
    ml2 = torch.zeros_like(ml)
    qa2 = torch.zeros_like(qa)
    cfh2 = torch.zeros_like(cfh)
    runs = A.atom_runs(tk.off, chunk)
    assert len(runs) > 1
    for n0, n1, e0, e1 in runs:
        rows = run_rows(N, n0, n1, e0, e1).to(device)
        qc = q.index_select(0, rows).contiguous()
        A.attn_fwd_run(n0, n1, e0, qc, off, cf, merged2, ml2, H, hd, T)
    for n0, n1, e0, e1 in runs:
        rows = run_rows(N, n0, n1, e0, e1).to(device)
        qc = q.index_select(0, rows).contiguous()
        dmc = dm.index_select(0, rows).contiguous()
        qac = torch.empty_like(qc)
        A.attn_bwd_run(n0, n1, e0, qc, off, dmc, merged2, ml2, cf, qac, cfh2, H, hd, T)
        qa2.index_copy_(0, rows, qac)
    torch.cuda.synchronize()
    assert torch.equal(merged, merged2)
    assert torch.equal(ml, ml2)
    assert torch.equal(qa, qa2)
    assert torch.equal(cfh, cfh2)


@pytest.mark.parametrize("beta,dead,chunk", [(0.0, False, 37), (1.0, False, 500), (0.0, True, 300),
                                             (1.0, True, 100000)])
def test_op_level_chunked(device, beta, dead, chunk):
    conf, tk = systems.config_tokens("c1")
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    print(f"[gpu] op-level chunked beta {beta} dead {dead} chunk {chunk}", flush=True)
    inp = systems.attention_inputs(tk, D, H, seed=6)
    rng = np.random.default_rng(7)
    T = tk.n_rows + (11 if dead else 0)
    qkv_h = np.concatenate([inp["qkv"], rng.standard_normal((T - tk.n_rows, 3 * D)).astype(np.float32)])
    out_adj_h = rng.standard_normal((T, D)).astype(np.float32)
    in_adj0 = rng.standard_normal((T, D)).astype(np.float32)
    cf_adj0 = rng.standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)
    temp = 0.9
    qkv = torch.from_numpy(qkv_h).to(device)
    cf = torch.from_numpy(tk.cf_seq).to(device)
    w_in, w_out, b_out = (torch.from_numpy(inp[k]).to(device) for k in ("w_in", "w_out", "b_out"))
    out_adj = torch.from_numpy(out_adj_h).to(device)
    t = A.Tokens(torch.from_numpy(tk.off).to(device), tk.n_atoms, dead)
    S = tk.slots

    calls = []

    def make_qkv(rows, r0, r1):
        calls.append((r0, r1))
        rows.copy_(qkv[r0:r1])

    ws1, ws2 = A.Workspace(device), A.Workspace(device)
    out1, out2 = torch.empty((T, D), device=device), torch.empty((T, D), device=device)
    A.attention(ws1, "a", out1, qkv, cf, w_out, b_out, t, S, H, hd, temp, True)
    A.attention_chunked(ws2, "a", out2, make_qkv, cf, w_out, b_out, t, tk.off, S, H, hd, temp, True, chunk)
    in1 = torch.from_numpy(in_adj0).to(device)
    in2 = in1.clone()
    ca1 = torch.from_numpy(cf_adj0).to(device)
    ca2 = ca1.clone()
    A.attention_bwd(ws1, "a", in1, ca1, out_adj, qkv, cf, w_in, w_out, t, S, H, hd, temp, beta)
    A.attention_bwd_chunked(ws2, "a", in2, ca2, out_adj, make_qkv, cf, w_in, w_out, t, tk.off, S, H, hd, temp, beta,
                            chunk)
    torch.cuda.synchronize()
    runs = A.atom_runs(tk.off, chunk)
    assert len(calls) == 2 * sum(1 + (e1 > e0) for _, _, e0, e1 in runs)
    assert torch.equal(ws1.peek2("a:merged"), ws2.peek2("a:merged"))
    assert torch.equal(ws1.peek2("a:ml"), ws2.peek2("a:ml"))
    o1, o2 = out1.cpu().numpy(), out2.cpu().numpy()
    i1, i2 = in1.cpu().numpy(), in2.cpu().numpy()
    c1, c2 = ca1.cpu().numpy(), ca2.cpu().numpy()
    # dmerged = out_adj W_out comes from a per-run GEMM, so everything after it
    # is held to a tolerance, with its bitwise agreement reported
    print(f"    out {rel(o2, o1):.1e} (bitwise {np.array_equal(o1, o2)}), in_adj {rel(i2, i1):.1e} "
          f"(bitwise {np.array_equal(i1, i2)}), cf_seq_adj {rel(c2, c1):.1e} (bitwise {np.array_equal(c1, c2)})",
          flush=True)
    assert rel(o2, o1) <= 1e-6 and rel(i2, i1) <= 1e-6 and rel(c2, c1) <= 1e-6
    # and both against the oracle
    rout, rm, rml = oracle.attention(qkv_h, tk.off, tk.cf_seq, inp["w_out"], inp["b_out"], H, hd, temp, dead=dead)
    rin, rca = oracle.attention_bwd(out_adj_h, qkv_h, tk.off, tk.cf_seq, inp["w_in"], inp["w_out"], rm, rml, H, hd,
                                    temp, cf_seq_adj=cf_adj0, in_adj=in_adj0, beta=beta, dead=dead)
    assert row_err(o2, rout) <= RTOL and row_err(i2, rin) <= RTOL and row_err(ca2.cpu().numpy(), rca) <= RTOL
    if dead:
        assert np.array_equal(i2[tk.n_rows:], (beta * in_adj0[tk.n_rows:]).astype(np.float32))
