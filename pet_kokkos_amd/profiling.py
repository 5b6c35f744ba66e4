"""A fixed workload for rocprofv3: K core attention fwd+bwd steps on one of
the benchmark configurations, preceded by a plain device copy of known size
(the calibration kernel that HBM byte counters are scaled by).

    python -m pet_kokkos_amd.profiling --config c3 --steps 20 --copy-mib 1024
    python -m pet_kokkos_amd.profiling --model c2 --steps 10

With ``--model`` the steps are whole energy+forces evaluations of the PET
model on that workload (C2: 648-atom water; C5: 32 structures) instead; with
``--gemm M,N,K`` one dense product C = A W^T (+ bias) on random operands, each
step once from fp32 A (pet_linear_fused_split) and once from its pair rows
(pet_linear_pair_rows, then pet_linear_fused_pairs), optionally keeping the
pre-activation (``--gemm-pre``).

Under ``rocprofv3 --kernel-trace --stats`` it gives each kernel's average
duration; under ``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``) each
kernel's HBM kilobytes per dispatch, with the copy's own reading of a known
``--copy-mib`` MiB read and write as the scale.
"""
from __future__ import annotations

import argparse
import json
import sys

import torch

from . import attention as A
from . import systems


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="c3", choices=sorted(systems.CONFIGS))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--rows", action="store_true",
                    help="also run the token norm (forward, backward) and the forces' edge term and fold each step")
    ap.add_argument("--model", choices=["c2", "c2-residual", "c5"], help="profile whole energy+forces evaluations instead")
    ap.add_argument("--gemm", metavar="M,N,K", help="profile one dense product instead")
    ap.add_argument("--gemm-pre", action="store_true", help="with --gemm: bias and kept pre-activation epilogue")
    ap.add_argument("--option", action="append", default=[], metavar="NAME=VALUE",
                    help="a library option (pet_attn_set_option by name, e.g. bwd_kernel=1), repeatable")
    args = ap.parse_args(argv)
    from . import _lib
    for o in args.option:
        name, _, value = o.partition("=")
        _lib.set_option(name, int(value))
    device = torch.device("cuda", 0)
    if args.model:
        return profile_model(args, device)
    if args.gemm:
        return profile_gemm(args, device)
    conf, tk = systems.config_tokens(args.config, seed=0)
    H, hd, D = conf.heads, conf.head_dim, conf.d_model
    N, S, T = tk.n_atoms, tk.slots, tk.n_rows
    g = torch.Generator(device=device)
    g.manual_seed(7)
    qkv = torch.randn((T, 3 * D), device=device, generator=g)
    dm = torch.randn((T, D), device=device, generator=g)
    off = torch.from_numpy(tk.off).to(device)
    cf = torch.from_numpy(tk.cf_seq).to(device)
    merged = torch.empty((T, D), device=device)
    ml = torch.empty((N * H * S, 2), device=device)
    qkv_adj = torch.empty((T, 3 * D), device=device)
    cfh = torch.empty((N, H, S), device=device)
    cf_adj = torch.zeros((N, S), device=device)
    n = args.copy_mib * (1 << 20) // 4
    src = torch.randn(n, device=device, generator=g)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)  # calibration: reads and writes copy_mib MiB
    torch.cuda.synchronize()
    rows = None
    if args.rows:
        from . import forces as F
        from . import layer as L
        cfgs = systems.CONFIGS[args.config]
        s = systems.build_structure(cfgs.structure, 0)
        pk = F.PackedEdges.from_host(systems.packed_edges(len(s.positions),
                                                          systems.neighbor_list(s, cfgs.cutoff), cfgs.cutoff,
                                                          cfgs.width), device)
        x4 = torch.randn((pk.n_edges, 4), device=device, generator=g)
        nw = torch.ones(D, device=device)
        y, gx = torch.empty_like(dm), torch.empty_like(dm)
        grad = torch.empty((pk.n_edges, 3), dtype=torch.float64, device=device)

        def rows():
            L.norm_rows(y, dm, nw, None)
            L.norm_rows_bwd(gx, y, dm, nw, False)
            F.edge_grad(pk, x4, None, cf_adj, cfgs.width, "cosine", grad)
            F.fold_edge_gradients(pk, N, grad, -1.0)
    for _ in range(args.steps):
        A.attn_fwd(qkv, off, cf, H, hd, merged=merged, ml=ml)
        A.attn_bwd(qkv, off, dm, merged, ml, cf, H, hd, cf_seq_adj=cf_adj, qkv_adj=qkv_adj, cfh=cfh)
        if rows:
            rows()
    torch.cuda.synchronize()
    print(json.dumps({"config": args.config, "steps": args.steps, "copy_mib": args.copy_mib, "N": N, "T": T, "S": S,
                      "D": D, "H": H}), flush=True)
    return 0


def profile_model(args, device):
    from .model import PetModel, ef_workload, structures_input
    h, w, comp, sts = ef_workload(args.model)
    m = PetModel(h, w, comp)
    x = structures_input(h, sts, device)
    src = torch.randn(args.copy_mib * (1 << 20) // 4, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    del src, dst
    out = m.compute(x, True)
    for _ in range(args.steps):
        m.compute(x, True, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"model": args.model, "steps": args.steps, "atoms": x.n_atoms, "edges": x.n_edges}), flush=True)
    return 0


def profile_gemm(args, device):
    from . import linear as L
    M, N, K = (int(v) for v in args.gemm.split(","))
    g = torch.Generator(device=device)
    g.manual_seed(3)
    A = torch.randn((M, K), device=device, generator=g)
    W = torch.randn((N, K), device=device, generator=g) / K ** 0.5
    b = torch.randn(N, device=device, generator=g)
    C = torch.empty((M, N), device=device)
    pre = torch.empty((M, N), device=device) if args.gemm_pre else None
    Ws = L.SplitWeights(W)
    src = torch.randn(args.copy_mib * (1 << 20) // 4, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    del src, dst
    kw = dict(bias=b, pre=pre) if args.gemm_pre else {}
    for _ in range(args.steps):
        L.fused(A, Ws, C, **kw)
        L.fused(L.PairRows(A), Ws, C, **kw)
    torch.cuda.synchronize()
    print(json.dumps({"gemm": [M, N, K], "steps": args.steps, "pre": args.gemm_pre}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
