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
PEAK_HBM = 8.0e12  # B/s


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-op-level", action="store_true", help="skip the op-level (with linears) timing")
    ap.add_argument("--cpu-reps", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the attention needs no communication; "
              "multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

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

    for _ in range(args.warmup):
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
    core_flops = alg["fwd_flops"] + alg["bwd_flops"]
    core_bytes = alg["fwd_bytes"] + alg["bwd_bytes"]
    bound_us = max(core_flops / PEAK_FP32_MFMA, core_bytes / PEAK_HBM) * 1e6
    bwd_mfma_bound = alg["bwd_flops"] / PEAK_FP32_MFMA >= alg["bwd_bytes"] / PEAK_HBM
    if bwd_mfma_bound:
        achieved = alg["bwd_flops"] / (bwd_avg * 1e-6) / 1e12
        roof = dict(kernel="attn_bwd_kernel<32> (+ attn_cf_adjoint_kernel)", bound="mfma", achieved=achieved,
                    peak=PEAK_FP32_MFMA / 1e12, unit="TFLOP/s", frac=achieved / (PEAK_FP32_MFMA / 1e12))
    else:
        achieved = alg["bwd_bytes"] / (bwd_avg * 1e-6) / 1e9
        roof = dict(kernel="attn_bwd_kernel", bound="hbm", achieved=achieved, peak=PEAK_HBM / 1e9, unit="GB/s",
                    frac=achieved / (PEAK_HBM / 1e9))
    roof["traffic"] = None
    tpath = os.path.join(ROOT, "profiles", f"attn_bwd_{args.config}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            roof["traffic"] = json.load(f).get("hbm_bytes_per_launch")

    extra = dict(
        fwd_us=fwd_avg, bwd_us=bwd_avg, fwd_us_min=min(fwd_us), bwd_us_min=min(bwd_us),
        step_us_median=statistics.median([a + b for a, b in zip(fwd_us, bwd_us)]),
        core_bound_us=bound_us, core_frac_of_roofline=bound_us / us_per_step,
        fwd_tflops=alg["fwd_flops"] / (fwd_avg * 1e-6) / 1e12,
        fwd_gbps=alg["fwd_bytes"] / (fwd_avg * 1e-6) / 1e9,
        bwd_gbps=alg["bwd_bytes"] / (bwd_avg * 1e-6) / 1e9,
        algorithmic=dict(sum_cnt2=alg["cnt2"], fwd_gflop=alg["fwd_flops"] / 1e9, bwd_gflop=alg["bwd_flops"] / 1e9,
                         fwd_mb=alg["fwd_bytes"] / 1e6, bwd_mb=alg["bwd_bytes"] / 1e6),
        wall_s=wall,
    )

    if not args.no_op_level:
        # attention() + attention_bwd(): the core plus the W_out / W_in linears (rocBLAS).
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
        extra["op_level_note"] = "attention()+attention_bwd(): core + W_out fwd, W_out^T and W_in^T GEMMs (rocBLAS)"

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
