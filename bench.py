#!/usr/bin/env python3
"""Benchmark of PET's neighbourhood attention forward + backward on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c3] [--no-cpu] [--no-op-level]

A step is one pass of the hot path over one batch: the core attention forward
(pet_attn_fwd: qkv -> merged, ml) and backward (pet_attn_bwd: -> qkv_adj, cfh,
cf_seq_adj) of one layer on the workload, inputs resident in HBM. The default
workload is BASELINE.json's north-star one, configs[2]: the 1728-atom diamond
(6x6x6 cells, a = 3.567 A, N(0, 0.02 A) jitter, cutoff 4.5 A, 71 tokens per
atom), d_model 256, 8 heads of 32, random-init weights, fp32.

Timing: W untimed warmup steps, then K steps between two synchronisations;
HIP events on the stream the kernels run on bracket every forward and every
backward call, which gives each kernel's average launch time. Printed: one
JSON line with value = microseconds per fwd+bwd (lower is better), the
roofline of the dominant kernel (the backward) against MI355X's fp32 matrix
peak, and the CPU baseline: the oracle (a restatement of the reference's
OpenMP host path) timed on this host's cores on the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "µs per attention fwd+bwd and ms per E+F eval (1 GPU), % of HBM/MFMA roofline"
PEAK_FP32_MFMA = 157.3e12  # FLOP/s, MI355X dense fp32 matrix
PEAK_BF16_MFMA = 2.5e15  # FLOP/s, MI355X dense bf16 (and fp16) matrix
# an fp32 product as six bf16 products (the split-fp32 scheme): fp32 FLOP/s
PEAK_SPLIT_FP32 = PEAK_BF16_MFMA / 6
# an fp32 product as three fp16 products (the fp16-pair scheme)
PEAK_PAIR_FP32 = PEAK_BF16_MFMA / 3
# the same on the 16x16x16 fp16 instruction, which issues at half the 16x16x32
# one's FLOP rate (measured on MI355X: 703 against 1236 TFLOP/s at best)
PEAK_PAIR16_FP32 = PEAK_BF16_MFMA / 2 / 3
# the short-K dense kernel: an fp32 product as five fp16 products (the
# weights in three parts, A in two)
PEAK_SHORTK_FP32 = PEAK_BF16_MFMA / 5
PEAK_HBM = 8.0e12  # B/s


def mixed_seconds(flops, split_share, pair_share=0.0, pair16_share=0.0, shortk_share=0.0):
    """Time at the matrix-core ceilings of the instructions that run: the
    split_share of the FLOPs as split-fp32 products on the bf16 matrix cores
    (2.5 PFLOP/s / 6), the pair_share as fp16-pair products (2.5 PFLOP/s / 3),
    the pair16_share as fp16-pair products on the 16x16x16 instruction
    (1.25 PFLOP/s / 3), the shortk_share as the short-K kernel's five fp16
    products (2.5 PFLOP/s / 5), the rest on the fp32 matrix cores
    (157.3 TFLOP/s)."""
    rest = 1.0 - split_share - pair_share - pair16_share - shortk_share
    return flops * (rest / PEAK_FP32_MFMA + split_share / PEAK_SPLIT_FP32 + pair_share / PEAK_PAIR_FP32
                    + pair16_share / PEAK_PAIR16_FP32 + shortk_share / PEAK_SHORTK_FP32)


def split_shares(plan, slots):
    """Shares (split, pair, pair16) of the forward's and the backward's FLOPs
    by the instructions that run them. Forward, scores and PV half each: with
    fwd_pair the scores as fp16 pairs on the 16x16x32 instruction, PV on it
    for key blocks taken two at a time and on the 16x16x16 one for a block
    alone (the own block, and an odd last one), else the scores split where
    fwd_split_scores. Backward, five products (scores, dP, dQ, dK, dV) a fifth
    each: with bwd_pair the scores and dP as fp16 pairs on the 16x16x32
    instruction and the other three on the 16x16x16 one, else dP split where
    bwd_split_dp."""
    if plan.get("streaming"):
        return (0.0, 0.0, 0.0), (0.0, 0.0, 0.0)
    if plan.get("fwd_pair"):
        nb = (slots + 15) // 16
        alone = nb - 2 * ((nb - 1) // 2)
        fwd = (0.0, 0.5 + 0.5 * (nb - alone) / nb, 0.5 * alone / nb)
    else:
        fwd = (0.5 * plan["fwd_split_scores"], 0.0, 0.0)
    bwd = (0.0, 0.4, 0.6) if plan.get("bwd_pair") else (0.2 * plan["bwd_split_dp"], 0.0, 0.0)
    return fwd, bwd


def bwd_kernel_name(plan, hd):
    if plan.get("streaming"):
        return "attn_bwd_stream_kernel"
    if plan.get("bwd_pair"):
        return f"attn_bwd_pair_kernel<{hd}, {plan['waves']}, false>"
    return f"attn_bwd_kernel<{hd}, 512>"


def algorithmic(tk, D, H):
    """FLOPs and bytes of the reference's accounting (tools/roofline.py:188-202),
    over real tokens."""
    import numpy as np
    cnt = tk.counts().astype(np.float64)
    cnt2 = float((cnt * cnt).sum())
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    stats = 4 * N * H * S * 2
    return dict(
        cnt2=cnt2,
        fwd_flops=4.0 * cnt2 * D, bwd_flops=10.0 * cnt2 * D,
        fwd_bytes=4.0 * (3 * T * D + T * D + N * S) + stats,
        bwd_bytes=4.0 * (3 * T * D + 2 * T * D + N * S + 3 * T * D + N * S * H) + stats,
    )


def _timed(fn, reps):
    """Average microseconds of fn() over reps calls, HIP events on the current stream."""
    import torch
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def time_rows(args, conf, tk, x, w_in, b_in, w_out, b_out, dm, off, cf, device):
    """The path's other rows on the same workload: the token norm (HBM-bound:
    bytes / time against 8 TB/s), the layer-level attention (norm, QKV linear,
    attention, output linear and their backward), and the forces' edge term and
    fold on the workload's own edge list."""
    import numpy as np
    import torch

    from pet_kokkos_amd import attention as A
    from pet_kokkos_amd import forces as F
    from pet_kokkos_amd import layer as L
    from pet_kokkos_amd import systems

    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    reps = max(10, args.steps // 2)
    out = {}
    nw = torch.ones(D, device=device)
    nb = torch.zeros(D, device=device)
    y = torch.empty_like(x)
    g = torch.empty_like(x)
    for name, bias in (("rmsnorm", None), ("layernorm", nb)):
        us_f = _timed(lambda: L.norm_rows(y, x, nw, bias), reps)
        us_b = _timed(lambda: L.norm_rows_bwd(g, dm, x, nw, bias is not None), reps)
        fb, bb = 2 * 4.0 * T * D, 3 * 4.0 * T * D
        out[name] = dict(fwd_us=us_f, bwd_us=us_b, fwd_gbps=fb / us_f / 1e3, bwd_gbps=bb / us_b / 1e3,
                         fwd_frac_hbm=fb / us_f / 1e3 / (PEAK_HBM / 1e9), bwd_frac_hbm=bb / us_b / 1e3 / (PEAK_HBM / 1e9))
    ws = A.Workspace(device)
    tkd = A.Tokens(off, N)
    o = torch.empty((T, D), device=device)
    tadj = torch.empty((T, D), device=device)
    ca = torch.zeros((N, S), device=device)
    out["layer_fwd_bwd_us"] = _timed(lambda: (
        L.attention_layer(ws, "b", o, x, nw, None, w_in, b_in, cf, w_out, b_out, tkd, S, H, hd, 1.0),
        L.attention_layer_bwd(ws, "b", tadj, ca, dm, x, nw, None, w_in, b_in, cf, w_out, tkd, S, H, hd, 1.0)), reps)
    out["layer_note"] = ("attention block of a PET layer: RMSNorm, QKV linear, attention, output linear, and the "
                         "backward (rebuilt norm and QKV, attention_bwd, norm backward into the token adjoint); "
                         "its dense products on the split-product kernel (fp32 accuracy on the 16-bit matrix cores: fp16 pairs "
                         "from K = 256, bf16 parts below)")
    cfgs = systems.CONFIGS[args.config]
    s = systems.build_structure(cfgs.structure, 0)
    pk = systems.packed_edges(len(s.positions), systems.neighbor_list(s, cfgs.cutoff), cfgs.cutoff, cfgs.width)
    E = len(pk.center)
    dpk = F.PackedEdges.from_host(pk, device)
    x4 = torch.randn((E, 4), device=device)
    csa = torch.randn((N, int(np.diff(pk.off).max()) + 1), device=device)
    grad = torch.empty((E, 3), dtype=torch.float64, device=device)
    us_e = _timed(lambda: F.edge_grad(dpk, x4, None, csa, cfgs.width, "cosine", grad), reps)
    us_f = _timed(lambda: F.fold_edge_gradients(dpk, N, grad, -1.0), reps)
    eb = E * (16 + 4 + 4 + 24 + 8 + 8 + 4 + 24)
    out["edge_grad"] = dict(us=us_e, edges=E, gbps=eb / us_e / 1e3)
    out["fold"] = dict(us=us_f, atoms=len(s.positions))
    out["other_configs"] = other_configs(device, reps)
    return out


def other_configs(device, reps):
    """Core fwd and bwd times of the ragged (C4) and batched (C5) workloads,
    with their fraction of the same roofline."""
    import torch

    from pet_kokkos_amd import _lib
    from pet_kokkos_amd import attention as A
    from pet_kokkos_amd import systems

    res = {}
    for name in ("c4", "c5"):
        conf, tk = systems.config_tokens(name, seed=0)
        H, hd, D = conf.heads, conf.head_dim, conf.d_model
        N, S, T = tk.n_atoms, tk.slots, tk.n_rows
        gen = torch.Generator(device=device)
        gen.manual_seed(3)
        qkv = torch.randn((T, 3 * D), device=device, generator=gen)
        dm = torch.randn((T, D), device=device, generator=gen)
        off = torch.from_numpy(tk.off).to(device)
        cf = torch.from_numpy(tk.cf_seq).to(device)
        merged = torch.empty((T, D), device=device)
        ml = torch.empty((N * H * S, 2), device=device)
        qa = torch.empty((T, 3 * D), device=device)
        cfh = torch.empty((N, H, S), device=device)
        ca = torch.zeros((N, S), device=device)
        f_us = _timed(lambda: A.attn_fwd(qkv, off, cf, H, hd, merged=merged, ml=ml), reps)
        b_us = _timed(lambda: A.attn_bwd(qkv, off, dm, merged, ml, cf, H, hd, cf_seq_adj=ca, qkv_adj=qa, cfh=cfh), reps)
        alg = algorithmic(tk, D, H)
        plan = _lib.describe(N, T, S, H, hd)
        fsh, bsh = split_shares(plan, S)
        bound = max(mixed_seconds(alg["fwd_flops"], *fsh) + mixed_seconds(alg["bwd_flops"], *bsh),
                    (alg["fwd_bytes"] + alg["bwd_bytes"]) / PEAK_HBM) * 1e6
        res[name] = dict(workload=conf.name, atoms=N, tokens=T, head_dim=hd, fwd_us=f_us, bwd_us=b_us,
                         bound_us=bound, frac_of_roofline=bound / (f_us + b_us), kernel_plan=plan)
        del qkv, dm, merged, ml, qa, cfh, ca
        torch.cuda.empty_cache()
    return res


def time_ef(device, reps, cpu: bool):
    """Energy+forces evaluations of the whole model (pet_model_compute): C2
    (configs[1], 648-atom water, d 128 / 4 heads / 2 x 2 layers / FFN 512) in
    both featurizers, and C5 (configs[4], 32 structures, d 512 / 8 heads of 64). ms per
    evaluation with inputs resident, the contraction roofline of its FLOPs
    (dense fp32 on the matrix cores: a lower bound that leaves out the
    HBM-bound elementwise passes) and, for C2, the CPU oracle (float32 torch on
    this host's cores) on the same structure."""
    import numpy as np
    import torch

    from pet_kokkos_amd import _lib
    from pet_kokkos_amd.model import PetModel, ef_flops, ef_workload, structures_input

    res, cpu_cases = {}, []
    # every GPU timing first, the CPU oracles after: a host thread pool left
    # spinning by an oracle run would slow the launches of the next timing
    for name in ("c2", "c2-residual", "c5"):
        h, w, comp, sts = ef_workload(name)
        m = PetModel(h, w, comp)
        x = structures_input(h, sts, device)
        cnt = np.diff(x.host.off).astype(np.float64) + 1
        fl = ef_flops(h, x.n_atoms, x.n_edges, float((cnt * cnt).sum()))
        n = max(3, reps // (5 if name != "c5" else 20))
        # contraction bound at the ceilings of the instructions that run: the
        # FLOPs this library's dense kernels launched in one evaluation, by
        # instruction class (pet_gemm_flop_tally: bf16 parts, fp16 pairs, the
        # short-K kernel's five fp16 products), the rest (rocBLAS's products,
        # the attention) on the fp32 matrix cores
        _lib.gemm_flop_tally(reset=True)
        o = m.compute(x, True)
        torch.cuda.synchronize()
        tal = _lib.gemm_flop_tally(reset=True)
        sh = {k: tal[k] / fl["forces"] for k in ("split", "pair", "shortk")}
        bound_ms = mixed_seconds(fl["forces"], sh["split"], sh["pair"], 0.0, sh["shortk"]) * 1e3
        e_ms = _timed(lambda: m.compute(x, False, out=o), n) / 1e3
        ef_ms = _timed(lambda: m.compute(x, True, out=o), n) / 1e3
        res[name] = dict(featurizer=h.featurizer, structures=len(sts), atoms=x.n_atoms, edges=x.n_edges,
                         d_pet=h.d_pet, heads=h.num_heads, ef_ms=ef_ms, energy_ms=e_ms, ef_tflop=fl["forces"] / 1e12,
                         ef_bound_ms=bound_ms, ef_frac_of_roofline=bound_ms / ef_ms,
                         ef_split_share=sh["split"], ef_pair_share=sh["pair"], ef_shortk_share=sh["shortk"],
                         ef_own_kernels_tflop=sum(tal.values()) / 1e12,
                         workspace_gb=m.workspace_bytes / 1e9, tier=m.last_tier,
                         pairs_scratch_gb=m.pairs_scratch_bytes / 1e9)
        if name == "c5":
            # the "wide" memory tier (qkv and the edge MLP's pre-activation
            # remade in the backward, the edge MLP over 64k-row chunks): the
            # same bits, a fresh model so its workspace is its own
            del m, o
            torch.cuda.empty_cache()
            m = PetModel(h, w, comp)
            with _lib.options(model_recompute=2):
                o = m.compute(x, True)
                wide_ms = _timed(lambda: m.compute(x, True, out=o), n) / 1e3
            res[name]["wide"] = dict(ef_ms=wide_ms, workspace_gb=m.workspace_bytes / 1e9, tier=m.last_tier)
        if name in ("c2", "c2-residual") and cpu:
            cpu_cases.append((name, h, w, comp, x.species.cpu().numpy(), x.host))
        del m, x, o
        torch.cuda.empty_cache()
    if cpu_cases:
        from oracle import pet_model as om
        for name, h, w, comp, sp, host in cpu_cases:
            om.evaluate(h, w, sp, host, comp, dtype=torch.float32)
            t = []
            for _ in range(2):
                c0 = time.perf_counter()
                om.evaluate(h, w, sp, host, comp, dtype=torch.float32)
                t.append(time.perf_counter() - c0)
            res[name]["cpu_ms"] = min(t) * 1e3
            res[name]["cpu_note"] = (f"oracle/pet_model.py in float32 torch on {torch.get_num_threads()} host "
                                     "threads, forces by autograd, best of 2 after a warmup")
    res["note"] = ("random-init PET-shaped models: feedforward featurizer (RMSNorm, SwiGLU, d_node 2 d_pet, "
                   "d_head 128) for c2 and c5, residual featurizer (LayerNorm, SiLU, d_node d_pet) for "
                   "c2-residual; neighbour list built on the host beforehand and not timed")
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--warmup-s", type=float, default=2.0, help="warm up for at least this many seconds")
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-op-level", action="store_true", help="skip the op-level (with linears) timing")
    ap.add_argument("--no-rows", action="store_true",
                    help="skip the timing of the path's other rows (token norm, layer level, forces' edge term)")
    ap.add_argument("--no-ef", action="store_true", help="skip the whole-model energy+forces timing (C2, C5)")
    ap.add_argument("--cpu-reps", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the attention needs no communication; "
              "multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from pet_kokkos_amd import _lib
    from pet_kokkos_amd import attention as A
    from pet_kokkos_amd import systems

    device = torch.device("cuda", 0)
    conf, tk = systems.config_tokens(args.config, seed=0)
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    gen = torch.Generator(device=device)
    gen.manual_seed(1234)
    x = torch.randn((T, D), device=device, generator=gen)
    w_in = torch.randn((3 * D, D), device=device, generator=gen) / D ** 0.5
    b_in = 0.1 * torch.randn((3 * D,), device=device, generator=gen)
    w_out = torch.randn((D, D), device=device, generator=gen) / D ** 0.5
    b_out = 0.1 * torch.randn((D,), device=device, generator=gen)
    qkv = torch.addmm(b_in, x, w_in.t()).contiguous()
    dm = torch.randn((T, D), device=device, generator=gen)
    off = torch.from_numpy(tk.off).to(device)
    cf = torch.from_numpy(tk.cf_seq).to(device)
    merged = torch.empty((T, D), device=device)
    ml = torch.empty((N * H * S, 2), device=device)
    qkv_adj = torch.empty((T, 3 * D), device=device)
    cfh = torch.empty((N, H, S), device=device)
    cf_adj = torch.zeros((N, S), device=device)

    def step(ev=None):
        if ev:
            ev[0].record()
        A.attn_fwd(qkv, off, cf, H, hd, merged=merged, ml=ml)
        if ev:
            ev[1].record()
        A.attn_bwd(qkv, off, dm, merged, ml, cf, H, hd, cf_seq_adj=cf_adj, qkv_adj=qkv_adj, cfh=cfh)
        if ev:
            ev[2].record()

    # W warmup steps, then more until --warmup-s seconds have passed (the
    # clocks settle; a short warmup left the first timed steps slower)
    w0 = time.perf_counter()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    while time.perf_counter() - w0 < args.warmup_s:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for k in range(args.steps):
        step(evs[k])
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(end)
    fwd_us = [e[0].elapsed_time(e[1]) * 1e3 for e in evs]
    bwd_us = [e[1].elapsed_time(e[2]) * 1e3 for e in evs]
    us_per_step = total_ms * 1e3 / args.steps
    alg = algorithmic(tk, D, H)
    fwd_avg, bwd_avg = statistics.fmean(fwd_us), statistics.fmean(bwd_us)
    plan = _lib.describe(N, T, S, H, hd)
    fsh, bsh = split_shares(plan, S)
    core_bytes = alg["fwd_bytes"] + alg["bwd_bytes"]
    # the core's bound at the ceilings of the instructions that run
    core_mfma_s = mixed_seconds(alg["fwd_flops"], *fsh) + mixed_seconds(alg["bwd_flops"], *bsh)
    bound_us = max(core_mfma_s, core_bytes / PEAK_HBM) * 1e6
    bwd_mfma_s = mixed_seconds(alg["bwd_flops"], *bsh)
    kname = bwd_kernel_name(plan, hd) + " (+ attn_cf_adjoint_kernel)"
    if bwd_mfma_s >= alg["bwd_bytes"] / PEAK_HBM:
        peak = alg["bwd_flops"] / bwd_mfma_s  # fp32-equivalent FLOP/s of the instruction mix
        achieved = alg["bwd_flops"] / (bwd_avg * 1e-6) / 1e12
        roof = dict(kernel=kname, bound="mfma", achieved=achieved,
                    peak=peak / 1e12, unit="TFLOP/s", frac=achieved / (peak / 1e12),
                    ceiling=f"fp32 matrix peak 157.3 TFLOP/s for {100 * (1 - sum(bsh)):.0f}% of the FLOPs, split-fp32 "
                            f"on the bf16 matrix cores (2.5 PFLOP/s / 6) for {100 * bsh[0]:.0f}%")
    else:
        achieved = alg["bwd_bytes"] / (bwd_avg * 1e-6) / 1e9
        roof = dict(kernel=kname, bound="hbm", achieved=achieved, peak=PEAK_HBM / 1e9, unit="GB/s",
                    frac=achieved / (PEAK_HBM / 1e9),
                    ceiling=f"HBM 8 TB/s; the matrix-core time at the ceilings of the instructions that run is "
                            f"{bwd_mfma_s * 1e6:.1f} us")
    roof["traffic"] = None
    tpath = os.path.join(ROOT, "profiles", f"attn_bwd_{args.config}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            roof["traffic"] = json.load(f).get("hbm_bytes_per_launch")

    steps_us = [a + b for a, b in zip(fwd_us, bwd_us)]
    extra = dict(
        fwd_us=fwd_avg, bwd_us=bwd_avg, fwd_us_min=min(fwd_us), bwd_us_min=min(bwd_us),
        fwd_us_median=statistics.median(fwd_us), bwd_us_median=statistics.median(bwd_us),
        step_us_median=statistics.median(steps_us), step_us_min=min(steps_us),
        core_bound_us=bound_us, core_frac_of_roofline=bound_us / us_per_step,
        core_bound_fp32_only_us=max((alg["fwd_flops"] + alg["bwd_flops"]) / PEAK_FP32_MFMA, core_bytes / PEAK_HBM) * 1e6,
        kernel_plan=plan,
        fwd_tflops=alg["fwd_flops"] / (fwd_avg * 1e-6) / 1e12,
        fwd_gbps=alg["fwd_bytes"] / (fwd_avg * 1e-6) / 1e9,
        bwd_gbps=alg["bwd_bytes"] / (bwd_avg * 1e-6) / 1e9,
        algorithmic=dict(sum_cnt2=alg["cnt2"], fwd_gflop=alg["fwd_flops"] / 1e9, bwd_gflop=alg["bwd_flops"] / 1e9,
                         fwd_mb=alg["fwd_bytes"] / 1e6, bwd_mb=alg["bwd_bytes"] / 1e6),
        wall_s=wall,
    )
    # the kernels' own access pattern with no arithmetic (pet_attn_access_floor,
    # head_dim 32): the floor their HBM traffic sets on this device
    if hd == 32 and S <= 128:
        lib = _lib.load()
        shp = _lib.Shape(N, T, S, H, hd, 0, lib.pet_attn_scale(hd, 1.0))
        mp, mlp = torch.empty_like(merged), torch.empty_like(ml)
        qap, cfhp = torch.empty_like(qkv_adj), torch.empty_like(cfh)
        st = torch.cuda.current_stream().cuda_stream
        import ctypes

        def floor_call(bwd):
            _lib.check(lib.pet_attn_access_floor(ctypes.byref(shp), bwd, qkv.data_ptr(), 3 * D, off.data_ptr(),
                                                 dm.data_ptr(), D, (merged if bwd else mp).data_ptr(), D,
                                                 mlp.data_ptr(), qap.data_ptr(), 3 * D, cfhp.data_ptr(), st),
                       "pet_attn_access_floor")
        fl = {}
        for bwd in (0, 1):
            for _ in range(5):
                floor_call(bwd)
            f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            f0.record()
            for _ in range(20):
                floor_call(bwd)
            f1.record()
            torch.cuda.synchronize()
            fl["bwd" if bwd else "fwd"] = f0.elapsed_time(f1) * 1e3 / 20
        extra["access_floor_us"] = fl
        extra["core_frac_of_access_floor"] = (fl["fwd"] + fl["bwd"]) / us_per_step
        extra["access_floor_note"] = ("pet_attn_access_floor: the fp16-pair kernels' grid, item order and bytes with "
                                      "no arithmetic; the floor their traffic sets on this device")
        del mp, mlp, qap, cfhp
    # the same step recorded once as a HIP graph and replayed K times: the
    # kernels and their bytes unchanged, the launches' host and queue overhead
    # gone (`value` stays the eager calls')
    try:
        gs = torch.cuda.Stream()
        gs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(gs):
            step()
            step()
        torch.cuda.current_stream().wait_stream(gs)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(5):
            graph.replay()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        g0.record()
        for _ in range(args.steps):
            graph.replay()
        g1.record()
        torch.cuda.synchronize()
        extra["graph_step_us"] = g0.elapsed_time(g1) * 1e3 / args.steps
        del graph
    except Exception as ex:  # a measurement aside: report, do not fail the bench
        extra["graph_step_us"] = None
        extra["graph_step_note"] = f"not recorded: {ex}"
    # the box's achievable streaming rate, for scale: a plain 1 GiB device copy
    # (read + write) timed the same way; the roofline stays against 8 TB/s
    src = torch.empty(1 << 28, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(10):
        dst.copy_(src)
    c1.record()
    torch.cuda.synchronize()
    copy_tbps = 2 * src.numel() * 4 * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e12
    extra["hbm_copy_tbps"] = copy_tbps
    extra["core_frac_of_copy_rate"] = core_bytes / (copy_tbps * 1e12) / (us_per_step * 1e-6)
    del src, dst

    if not args.no_op_level:
        # attention() + attention_bwd(): the core plus the W_out / W_in linears.
        ws = A.Workspace(device)
        tkd = A.Tokens(off, N)
        out = torch.empty((T, D), device=device)
        in_adj = torch.empty((T, D), device=device)
        cf_adj2 = torch.zeros((N, S), device=device)

        def op_step():
            A.attention(ws, "bench", out, qkv, cf, w_out, b_out, tkd, S, H, hd, 1.0, True)
            A.attention_bwd(ws, "bench", in_adj, cf_adj2, dm, qkv, cf, w_in, w_out, tkd, S, H, hd, 1.0, 0.0)

        for _ in range(max(3, args.warmup // 2)):
            op_step()
        torch.cuda.synchronize()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = max(10, args.steps // 2)
        s0.record()
        for _ in range(reps):
            op_step()
        s1.record()
        torch.cuda.synchronize()
        extra["op_level_us"] = s0.elapsed_time(s1) * 1e3 / reps
        # its bound: the core's (the larger of its HBM and matrix-core times)
        # plus each dense product's larger of its own HBM bytes and its FLOPs
        # at the ceiling of the instruction it runs on: the output linear
        # out = merged W_out^T + b (2 T D^2 FLOP; merged and out, 8 T D + 4 D^2
        # bytes), dmerged = out_adj W_out (2 T D^2; 8 T D + 4 D^2) and the input
        # adjoint qkv_adj W_in (6 T D^2; 16 T D + 12 D^2), each on the
        # split-product kernel: fp16 pairs from K = 256, bf16 parts below
        def gemm_s(flops, nbytes, k):
            pair = k >= 256
            return max(nbytes / PEAK_HBM, mixed_seconds(flops, 0.0 if pair else 1.0, 1.0 if pair else 0.0))
        gemms = [gemm_s(2.0 * T * D * D, 8.0 * T * D + 4.0 * D * D, D),
                 gemm_s(2.0 * T * D * D, 8.0 * T * D + 4.0 * D * D, D),
                 gemm_s(6.0 * T * D * D, 16.0 * T * D + 12.0 * D * D, 3 * D)]
        extra["op_level_bound_us"] = (bound_us * 1e-6 + sum(gemms)) * 1e6
        extra["op_level_bound_parts_us"] = dict(core=bound_us, out_linear=gemms[0] * 1e6, dmerged=gemms[1] * 1e6,
                                                in_adj=gemms[2] * 1e6)
        extra["op_level_frac_of_roofline"] = extra["op_level_bound_us"] / extra["op_level_us"]
        extra["op_level_note"] = ("attention()+attention_bwd(): core + the output linear (split-product kernel, W_out "
                                  "split as it is staged, bias in its epilogue), dmerged = out_adj W_out and the input "
                                  "adjoint (split-product kernel, W_out^T and W_in^T split into the workspace)")

    if not args.no_rows:
        extra["rows"] = time_rows(args, conf, tk, x, w_in, b_in, w_out, b_out, dm, off, cf, device)
    if not args.no_ef:
        extra["ef"] = time_ef(device, max(10, args.steps // 2), not args.no_cpu)

    cpu = None
    if not args.no_cpu:
        import oracle
        qkv_h, dm_h = qkv.cpu().numpy(), dm.cpu().numpy()
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))

        def cpu_step():
            m, l = oracle.attn_fwd(qkv_h, tk.off, tk.cf_seq, H, hd)
            oracle.attn_bwd(qkv_h, tk.off, dm_h, m, l, tk.cf_seq, H, hd)

        cpu_step()  # warmup
        times = []
        for _ in range(args.cpu_reps):
            c0 = time.perf_counter()
            cpu_step()
            times.append(time.perf_counter() - c0)
        cpu = dict(value=min(times) * 1e6, unit="us per fwd+bwd", cores=threads, kind="port",
                   sample=f"the full {conf.name} core fwd+bwd, best of {args.cpu_reps} after 1 warmup "
                          f"(OpenMP over (atom, head, slot) like the reference's host build; {threads} threads)")
        extra["gpu_speedup_vs_cpu"] = cpu["value"] / us_per_step

    line = {
        "metric": METRIC,
        "value": us_per_step,
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": us_per_step / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": f"{args.config} {conf.name}: core attention fwd+bwd (qkv -> merged, ml -> qkv_adj, "
                               f"cf_seq_adj), one layer", "atoms": N, "tokens": T, "slots": S, "d_model": D,
                   "heads": H, "head_dim": hd, "tokens_per_atom": [int(tk.counts().min()), int(tk.counts().max())],
                   "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
