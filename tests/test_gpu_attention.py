"""Parity of the HIP attention (through the C ABI) with the CPU oracle and the
golden vectors, on an MI355X.

Tolerance: every element of every attention output and
gradient within 1e-5 relative of the oracle's fp32 result, with an absolute
floor tied to the scale of its row (|gpu - ref| <= 1e-5 (|ref| + F_row)), for
the cf adjoint and the saved max the scale of the terms they are differences
of (tests/parity.py states the rules and why), and the same against the
oracle's fp64 twin. Measured on MI355X (C1-C4, the golden vectors): at most
1.6e-6 against either. Run to run the kernels are
bit-identical.
"""
from __future__ import annotations

import glob
import os
import sys

import numpy as np
import pytest
import torch

import oracle
from parity import RTOL, attention_errors, row_err
from pet_kokkos_amd import attention as A
from pet_kokkos_amd import systems

pytestmark = pytest.mark.gpu

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "attn_*.npz")))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    den = max(np.abs(b).max(), 1e-30) if b.size else 1.0
    return np.abs(a - b).max() / den if a.size else 0.0


def dev(x, device, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def gpu_fwd_bwd(device, off, cf_seq, qkv, dm, H, hd, temperature=1.0, dead=False, cf_adj0=None):
    N = len(off) - 1
    q, g, cf = dev(qkv, device), dev(dm, device), dev(cf_seq, device)
    o = dev(off, device, torch.int32)
    merged, ml = A.attn_fwd(q, o, cf, H, hd, temperature, dead=dead)
    start = None if cf_adj0 is None else dev(cf_adj0, device)
    qa, ca, cfh = A.attn_bwd(q, o, g, merged, ml, cf, H, hd, temperature, cf_seq_adj=start, dead=dead)
    torch.cuda.synchronize()
    # cfh [N, H, S] -> the oracle's (the reference's) [N*S, H]
    cfh = cfh.permute(0, 2, 1).reshape(N * cf_seq.shape[1], H)
    return [t.cpu().numpy() for t in (merged, ml, qa, ca, cfh)]


def check_against_oracle(device, name, off, cf_seq, qkv, dm, H, hd, temperature=1.0, dead=False, T=None, f64=True):
    say(f"[gpu] {name}: N={len(off) - 1} T={qkv.shape[0]} S={cf_seq.shape[1]} H={H} hd={hd}")
    m, ml, qa, ca, cfh = gpu_fwd_bwd(device, off, cf_seq, qkv, dm, H, hd, temperature, dead)
    sc = oracle.scale(hd, temperature)
    for dt in ((np.float32, np.float64) if f64 else (np.float32,)):
        rm, rml = oracle.attn_fwd(qkv, off, cf_seq, H, hd, temperature, dead=dead, dtype=dt)
        rqa, rca, rcfh = oracle.attn_bwd(qkv, off, dm, rm, rml, cf_seq, H, hd, temperature, dead=dead, dtype=dt)
        errs = attention_errors(off, cf_seq, qkv, dm, H, hd, m, qa, ca, cfh, (rm, rqa, rca, rcfh), sc, ml, rml)
        say(f"     vs {np.dtype(dt).name} oracle:", {k: f"{v:.2e}" for k, v in errs.items()})
        for k, v in errs.items():
            assert v <= RTOL, f"{name}: {k} off by {v:.3e} (element-wise, floored) against the {np.dtype(dt).name} oracle"
    return m, ml, qa, ca, cfh


def random_case(counts, H, hd, seed=0, cf_kind="random", extra=0):
    base = systems.tokens_from_counts(counts, seed=seed, cf_kind=cf_kind)
    tk = systems.tokens_from_counts(counts, seed=seed, cf_kind=cf_kind, slots=base.slots + extra)
    rng = np.random.default_rng(seed + 7)
    D = H * hd
    qkv = rng.standard_normal((tk.n_rows, 3 * D)).astype(np.float32)
    dm = rng.standard_normal((tk.n_rows, D)).astype(np.float32)
    return tk, qkv, dm


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_golden_vectors(device, path):
    g = np.load(path)
    H, hd, temp = int(g["heads"]), int(g["head_dim"]), float(g["temperature"])
    say(f"[gpu] golden {os.path.basename(path)}")
    m, ml, qa, ca, cfh = gpu_fwd_bwd(device, g["off"], g["cf_seq"], g["qkv"], g["dmerged"], H, hd, temp)
    errs = attention_errors(g["off"], g["cf_seq"], g["qkv"], g["dmerged"], H, hd, m, qa, ca, cfh,
                            (g["merged"], g["qkv_adj"], g["cf_seq_adj"], g["cfh"]), float(g["scale"]), ml, g["ml"])
    say("     vs the fp64 brute force:", {k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v <= RTOL, k


@pytest.mark.parametrize("cfg", ["c1", "c2", "c4", "c3", "c5"])
def test_configs(device, cfg):
    conf, tk = systems.config_tokens(cfg)
    rng = np.random.default_rng(3)
    if cfg == "c5":  # 32 structures, 510k token rows at d 512: qkv drawn directly
        qkv = rng.standard_normal((tk.n_rows, 3 * conf.d_model), dtype=np.float32)
    else:
        qkv = systems.attention_inputs(tk, conf.d_model, conf.heads, seed=1)["qkv"]
    dm = rng.standard_normal((tk.n_rows, conf.d_model), dtype=np.float32)
    check_against_oracle(device, f"config {cfg} ({conf.name})", tk.off, tk.cf_seq, qkv, dm, conf.heads,
                         conf.head_dim, f64=cfg != "c5")


@pytest.mark.parametrize("hd", [16, 32, 48, 64, 80, 96, 112, 128])
def test_head_dims(device, hd):
    counts = [0, 15, 16, 31, 47, 5, 60, 33]
    tk, qkv, dm = random_case(counts, 2, hd, seed=hd, cf_kind="zeros", extra=2)
    check_against_oracle(device, f"head_dim {hd}", tk.off, tk.cf_seq, qkv, dm, 2, hd, temperature=0.8)


@pytest.mark.parametrize("hd,top", [(16, 255), (32, 200), (64, 140), (80, 120), (128, 70)])
def test_many_slots(device, hd, top):
    # many query blocks (past 8: the 1024-thread kernels; the lean LDS layouts)
    lib = A._lib.load()
    counts = [top, 3, top // 2, min(top, 130)]
    tk, qkv, dm = random_case(counts, 2, hd, seed=top, cf_kind="random")
    assert tk.slots <= lib.pet_attn_max_slots(hd)
    check_against_oracle(device, f"many slots hd {hd} S {tk.slots}", tk.off, tk.cf_seq, qkv, dm, 2, hd)


def test_max_slots(device):
    # the LDS-staged kernels' envelope; past it (and for head_dims not a
    # multiple of 16) the streaming kernels run (tests/test_gpu_stream.py)
    lib = A._lib.load()
    say(f"[gpu] max slots by head_dim: " + ", ".join(f"{h}:{lib.pet_attn_max_slots(h)}" for h in
                                                    (16, 32, 48, 64, 80, 96, 112, 128)))
    assert lib.pet_attn_max_slots(24) == 0
    assert 64 <= lib.pet_attn_max_slots(128) < 256 and lib.pet_attn_max_slots(16) == 256


def test_edge_cases(device):
    # isolated atoms, block boundaries, cf = 0 keys and queries, padding slots
    counts = [0, 0, 1, 14, 15, 16, 17, 31, 32, 33, 63, 0]
    tk, qkv, dm = random_case(counts, 4, 32, seed=5, cf_kind="zeros", extra=5)
    check_against_oracle(device, "edge cases", tk.off, tk.cf_seq, qkv, dm, 4, 32)


def test_dead_rows(device):
    tk, qkv, dm = random_case([10, 22, 5], 2, 32, seed=8)
    T = tk.n_rows + 9
    rng = np.random.default_rng(1)
    qkv = np.concatenate([qkv, rng.standard_normal((9, qkv.shape[1])).astype(np.float32)])
    dm = np.concatenate([dm, rng.standard_normal((9, dm.shape[1])).astype(np.float32)])
    m, _, qa, _, _ = check_against_oracle(device, "dead rows", tk.off, tk.cf_seq, qkv, dm, 2, 32, dead=True)
    assert np.all(m[tk.n_rows:] == 0) and np.all(qa[tk.n_rows:] == 0)
    assert T == m.shape[0]


def test_bit_identical_repeats(device):
    conf, tk = systems.config_tokens("c1")
    inp = systems.attention_inputs(tk, conf.d_model, conf.heads, seed=2)
    dm = np.random.default_rng(4).standard_normal((tk.n_rows, conf.d_model)).astype(np.float32)
    say("[gpu] bitwise repeats c1")
    first = gpu_fwd_bwd(device, tk.off, tk.cf_seq, inp["qkv"], dm, conf.heads, conf.head_dim)
    for _ in range(3):
        again = gpu_fwd_bwd(device, tk.off, tk.cf_seq, inp["qkv"], dm, conf.heads, conf.head_dim)
        for a, b in zip(first, again):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("hd", [32, 64, 96, 128])
def test_split_products_as_accurate_as_fp32(device, hd):
    # Where head_dim is a multiple of 32 the forward's scores run on the bf16
    # matrix cores with each fp32 operand split into three exact bf16 parts;
    # the option split = 0 keeps them on the fp32 matrix cores. Both must meet the
    # tolerance, and the split one at an error no larger than the fp32 one's
    # order (measured: 1.0e-7 against 1.9e-7 of sum |a b| per product).
    counts = [0, 15, 16, 31, 47, 5, 60, 33, 70, 71]
    tk, qkv, dm = random_case(counts, 2, hd, seed=100 + hd, cf_kind="random")
    rm, rml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, hd, 1.0)
    out = {}
    for mode in ("0", "1"):
        say(f"[gpu] split products hd {hd} split={mode}")
        with A._lib.options(split=int(mode)):
            out[mode] = check_against_oracle(device, f"split={mode} hd {hd}", tk.off, tk.cf_seq, qkv, dm, 2, hd)
    e0, e1 = row_err(out["0"][0], rm), row_err(out["1"][0], rm)
    say(f"    merged error: fp32 products {e0:.2e}, split {e1:.2e}")
    assert e1 <= max(4 * e0, 1e-6)
    if hd == 32:  # the split kernels are the ones taken there: their rounding differs
        assert not np.array_equal(out["0"][0], out["1"][0])
        assert not np.array_equal(out["0"][2], out["1"][2])


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("vlds,nbuf", [(1, 2), (1, 1), (2, 2), (2, 1)])
@pytest.mark.parametrize("split", ["1", "0"])
def test_backward_layouts(device, hd, vlds, nbuf, split):
    # Every LDS layout of the backward, forced (option bwd_vlds: 1 V staged,
    # 2 from global memory; bwd_nbuf: tile buffers), with the split
    # dP (V staged split, head_dim 32) and without: the pipelined two-buffer
    # step loop and the two-barrier one-buffer loop, on ragged atoms.
    counts = [0, 15, 16, 31, 47, 5, 60, 33, 70]
    tk, qkv, dm = random_case(counts, 2, hd, seed=200 + hd + 10 * vlds + nbuf, cf_kind="random")
    with A._lib.options(bwd_vlds=vlds, bwd_nbuf=nbuf, split=int(split)):
        check_against_oracle(device, f"backward layout vlds {vlds} nbuf {nbuf} split {split} hd {hd}", tk.off,
                             tk.cf_seq, qkv, dm, 2, hd)


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("qk,v,g,spread", [(1.0, 1.0, 1.0, 0.0), (0.05, 1e3, 1e-7, 0.0), (0.5, 1e-4, 3e4, 0.0),
                                            (0.5, 1.0, 1.0, 3.0)])
def test_pair_backward_scales(device, qk, v, g, spread, hd):
    # The fp16-pair kernels (the default at head_dim 32 and 64): the backward puts each item's
    # largest |Q|, |K|, |V|, |dO| at 2^15 by powers of two and bounds dS
    # from them: V and dO far from unit scale, and V and dO rows spread over
    # 10^+-spread within an item, must meet the same bar against the oracle.
    # (Q and K stay moderate: scores of hundreds make exp amplify any fp32
    # rounding of them, a conditioning no product order escapes.)
    counts = [0, 15, 16, 31, 47, 5, 60, 33, 70, 79]
    tk, qkv, dm = random_case(counts, 2, hd, seed=300 + int(spread), cf_kind="random")
    rng = np.random.default_rng(11)
    D = 2 * hd
    qkv[:, :2 * D] *= qk
    qkv[:, 2 * D:] *= v * 10.0 ** rng.uniform(-spread, spread, (qkv.shape[0], 1))
    dm = (dm * g * 10.0 ** rng.uniform(-spread, spread, (dm.shape[0], 1))).astype(np.float32)
    qkv = qkv.astype(np.float32)
    plan = A._lib.describe(tk.n_atoms, tk.n_rows, tk.slots, 2, hd)
    assert plan["bwd_pair"] == 1 and plan["fwd_pair"] == 1
    check_against_oracle(device, f"pair kernels hd {hd} qk x{qk} v x{v} dO x{g} spread 1e+-{spread}", tk.off,
                         tk.cf_seq, qkv, dm, 2, hd)


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("spread", [4.0, 8.0])
def test_pair_qk_row_spread(device, spread, hd):
    # Q and K token rows spread over 10^-spread .. 1 within every item (each
    # row's own factor, Q's and K's independent), so the pair kernels' per-item
    # (backward) and per-block (forward) scales meet rows far below the
    # largest: every score stays at most |q||k| sc of unit rows (moderate), while
    # the smallest rows sit 2^-13 (spread 4) and 2^-27 (spread 8) below their
    # item's largest, near the 2^-29 down to which a pair keeps 22 bits.
    counts = [0, 15, 16, 31, 47, 5, 60, 33, 70, 79]
    tk, qkv, dm = random_case(counts, 2, hd, seed=700 + int(spread) + hd, cf_kind="random")
    rng = np.random.default_rng(int(spread) * 7 + hd)
    D = 2 * hd
    T = qkv.shape[0]
    qkv[:, :D] *= 10.0 ** rng.uniform(-spread, 0.0, (T, 1))
    qkv[:, D:2 * D] *= 10.0 ** rng.uniform(-spread, 0.0, (T, 1))
    qkv = qkv.astype(np.float32)
    plan = A._lib.describe(tk.n_atoms, tk.n_rows, tk.slots, 2, hd)
    assert plan["bwd_pair"] == 1 and plan["fwd_pair"] == 1
    check_against_oracle(device, f"pair kernels hd {hd}: Q, K rows spread over 1e-{spread:.0f}..1", tk.off,
                         tk.cf_seq, qkv, dm, 2, hd)


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("fwd,bwd", [(0, 0), (1, 1), (0, 1), (1, 0)])
def test_pair_and_staged_kernels(device, fwd, bwd, hd):
    # The head_dim-32 and -64 kernels in each combination (option fwd_kernel / bwd_kernel:
    # 0 the fp16-pair kernels, 1 the staged split-bf16 forward and the
    # tile-exchange backward) on ragged atoms, each bit-identical when repeated.
    counts = [0, 15, 16, 31, 47, 5, 60, 33, 70]
    tk, qkv, dm = random_case(counts, 3, hd, seed=400, cf_kind="random")
    with A._lib.options(fwd_kernel=fwd, bwd_kernel=bwd):
        plan = A._lib.describe(tk.n_atoms, tk.n_rows, tk.slots, 3, hd)
        assert plan["fwd_pair"] == (fwd == 0) and plan["bwd_pair"] == (bwd == 0)
        first = check_against_oracle(device, f"hd {hd}: forward kernel {fwd}, backward kernel {bwd}", tk.off,
                                     tk.cf_seq, qkv, dm, 3, hd)
        again = gpu_fwd_bwd(device, tk.off, tk.cf_seq, qkv, dm, 3, hd)
    for a, b in zip(first, again):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_cf_adjoint_accumulates(device):
    tk, qkv, dm = random_case([12, 40, 7], 2, 32, seed=6)
    start = np.random.default_rng(0).standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)
    say("[gpu] cf adjoint accumulates")
    _, _, _, ca0, _ = gpu_fwd_bwd(device, tk.off, tk.cf_seq, qkv, dm, 2, 32)
    _, _, _, ca1, _ = gpu_fwd_bwd(device, tk.off, tk.cf_seq, qkv, dm, 2, 32, cf_adj0=start)
    assert np.array_equal(ca1, (start + ca0).astype(np.float32))


def test_strided_views_and_stream(device):
    # leading dimensions above the widths (views into wider buffers), on a side stream
    tk, qkv, dm = random_case([20, 9, 33], 2, 32, seed=12)
    D = 64
    T = tk.n_rows
    say("[gpu] strided views")
    big = torch.zeros((T, 3 * D + 8), device=device)
    big[:, :3 * D] = dev(qkv, device)
    q = big[:, :3 * D]
    gbig = torch.zeros((T, D + 4), device=device)
    gbig[:, :D] = dev(dm, device)
    g = gbig[:, :D]
    cfbig = torch.zeros((tk.n_atoms, tk.slots + 4), device=device)
    cfbig[:, :tk.slots] = dev(tk.cf_seq, device)
    cf = cfbig[:, :tk.slots]
    mbig = torch.full((T, D + 12), 7.0, device=device)
    m = mbig[:, :D]
    qabig = torch.full((T, 3 * D + 4), 7.0, device=device)
    o = dev(tk.off, device, torch.int32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _, ml = A.attn_fwd(q, o, cf, 2, 32, merged=m)
        qa, ca, _ = A.attn_bwd(q, o, g, m, ml, cf, 2, 32, qkv_adj=qabig[:, :3 * D])
    torch.cuda.synchronize()
    rm, rml = oracle.attn_fwd(qkv, tk.off, tk.cf_seq, 2, 32)
    rqa, rca, _ = oracle.attn_bwd(qkv, tk.off, dm, rm, rml, tk.cf_seq, 2, 32)
    assert row_err(m.cpu().numpy(), rm) <= RTOL
    assert row_err(qa.cpu().numpy(), rqa) <= RTOL
    assert row_err(ca.cpu().numpy(), rca) <= RTOL
    assert torch.all(mbig[:, D:] == 7.0) and torch.all(qabig[:, 3 * D:] == 7.0)


@pytest.mark.parametrize("cfg", ["c1", "c3"])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_op_level_attention(device, beta, cfg):
    # attention()/attention_bwd() with the output and input linears, as the
    # reference's feedforward (beta 0) and residual (beta 1) featurizers call them,
    # on C1 and at C3's full size.
    conf, tk = systems.config_tokens(cfg)
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    inp = systems.attention_inputs(tk, D, H, seed=5)
    rng = np.random.default_rng(9)
    in_adj0 = rng.standard_normal((tk.n_rows, D)).astype(np.float32)
    cf_adj0 = rng.standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)
    temp = 1.3
    say(f"[gpu] op level {cfg} beta={beta}")
    ws = A.Workspace(device)
    t = A.Tokens(dev(tk.off, device, torch.int32), tk.n_atoms)
    out = torch.empty((tk.n_rows, D), device=device)
    qkv, cf = dev(inp["qkv"], device), dev(tk.cf_seq, device)
    w_in, w_out, b_out = dev(inp["w_in"], device), dev(inp["w_out"], device), dev(inp["b_out"], device)
    A.attention(ws, "L0.a0", out, qkv, cf, w_out, b_out, t, tk.slots, H, hd, temp, True)
    in_adj = dev(in_adj0, device)
    cf_adj = dev(cf_adj0, device)
    A.attention_bwd(ws, "L0.a0", in_adj, cf_adj, dev(inp["out_adj"], device), qkv, cf, w_in, w_out, t, tk.slots, H,
                    hd, temp, beta)
    torch.cuda.synchronize()
    rout, rm, rml = oracle.attention(inp["qkv"], tk.off, tk.cf_seq, inp["w_out"], inp["b_out"], H, hd, temp)
    rin, rca = oracle.attention_bwd(inp["out_adj"], inp["qkv"], tk.off, tk.cf_seq, inp["w_in"], inp["w_out"], rm, rml,
                                    H, hd, temp, cf_seq_adj=cf_adj0, in_adj=in_adj0, beta=beta)
    e = dict(out=row_err(out.cpu().numpy(), rout), in_adj=row_err(in_adj.cpu().numpy(), rin),
             cf_seq_adj=row_err(cf_adj.cpu().numpy(), rca))
    say("    ", {k: f"{v:.2e}" for k, v in e.items()})
    for k, v in e.items():
        assert v <= RTOL, k


def test_backward_before_forward_raises(device):
    ws = A.Workspace(device)
    with pytest.raises(RuntimeError):
        ws.peek2("nothing:merged")


def test_op_level_dead_rows_block_pairs(device):
    # attention_bwd() at C3's size (where the backward writes qkv_adj as block
    # pairs into the input adjoint's product) with 4096 capacity rows past the
    # tokens: the real rows as the oracle's without them, the dead rows of
    # in_adj exactly beta times their value before (a zero qkv adjoint there)
    conf, tk = systems.config_tokens("c3")
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    inp = systems.attention_inputs(tk, D, H, seed=11)
    extra, T = 4096, tk.n_rows + 4096
    rng = np.random.default_rng(12)
    pad = lambda a: np.concatenate([a, rng.standard_normal((extra, a.shape[1])).astype(np.float32)])
    qkv_d, oadj_d = pad(inp["qkv"]), pad(inp["out_adj"])
    in_adj0 = rng.standard_normal((T, D)).astype(np.float32)
    cf_adj0 = rng.standard_normal((tk.n_atoms, tk.slots)).astype(np.float32)
    say("[gpu] op level c3 with 4096 dead rows, beta=1")
    ws = A.Workspace(device)
    t = A.Tokens(dev(tk.off, device, torch.int32), tk.n_atoms, dead=True)
    out = torch.empty((T, D), device=device)
    qkv, cf = dev(qkv_d, device), dev(tk.cf_seq, device)
    w_in, w_out, b_out = dev(inp["w_in"], device), dev(inp["w_out"], device), dev(inp["b_out"], device)
    A.attention(ws, "L0.a0", out, qkv, cf, w_out, b_out, t, tk.slots, H, hd, 1.0, True)
    in_adj, cf_adj = dev(in_adj0, device), dev(cf_adj0, device)
    A.attention_bwd(ws, "L0.a0", in_adj, cf_adj, dev(oadj_d, device), qkv, cf, w_in, w_out, t, tk.slots, H, hd, 1.0,
                    1.0)
    torch.cuda.synchronize()
    got = in_adj.cpu().numpy()
    assert np.array_equal(got[tk.n_rows:], in_adj0[tk.n_rows:])
    _, rm, rml = oracle.attention(inp["qkv"], tk.off, tk.cf_seq, inp["w_out"], inp["b_out"], H, hd, 1.0)
    rin, rca = oracle.attention_bwd(inp["out_adj"], inp["qkv"], tk.off, tk.cf_seq, inp["w_in"], inp["w_out"], rm, rml,
                                    H, hd, 1.0, cf_seq_adj=cf_adj0, in_adj=in_adj0[: tk.n_rows], beta=1.0)
    e = dict(in_adj=row_err(got[: tk.n_rows], rin), cf_seq_adj=row_err(cf_adj.cpu().numpy(), rca))
    say("    ", {k: f"{v:.2e}" for k, v in e.items()})
    for k, v in e.items():
        assert v <= RTOL, k
