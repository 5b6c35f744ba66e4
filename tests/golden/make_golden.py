"""Writes the golden vectors of PET's neighbourhood attention (tests/golden/attn_*.npz).

    python tests/golden/make_golden.py

The expected values come from an independent brute force in float64 torch --
per atom and head, the full scores matrix, torch.softmax, and torch.autograd
for every gradient -- not from the oracle or the HIP kernels they check. The
semantics are the reference's (peterspackman/pet-kokkos src/attention.cpp:1-16,
:217-248, :1560-1568): keys with cf <= 0 are left out, a query on a cf <= 0
edge outputs zeros and takes no gradient, the saved statistics are
(max score, 1 / sum of exp(score - max)) with (-1e30, 0) for a slot with no
live query. cfh[n S + k, h] is d loss / d (log cf_k) of head h;
cf_seq_adj[n, k] = sum_h cfh / cf_k. The loss is sum(merged * dmerged).

Inputs are float32 values (qkv, dmerged ~ N(0, 1), cf in (0.05, 1] with some
exact zeros), seeded; the brute force runs on them widened to float64 with the
kernels' float32 scale.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from pet_kokkos_amd.systems import tokens_from_counts  # noqa: E402

CASES = {
    # name: (edge counts per atom, heads, head_dim, temperature, cf kind, extra slots, seed)
    "small_hd16": ([0, 2, 14, 15, 16, 30, 5, 1], 2, 16, 1.0, "zeros", 3, 1),
    "ragged_hd32": ([40, 7, 31, 32, 47, 12, 0, 63], 3, 32, 0.7, "zeros", 0, 2),
    "ones_hd48": ([9, 20, 33], 2, 48, 1.0, "ones", 1, 3),
    "wide_hd64": ([70, 70, 3], 2, 64, 1.3, "random", 0, 4),
}


def kernel_scale(hd: int, temperature: float) -> float:
    return float(np.float32(1.0 / (np.sqrt(np.float64(hd)) * temperature)))


def brute_force(qkv, off, cf_seq, dmerged, H, hd, sc):
    N, S = cf_seq.shape
    D = H * hd
    T = qkv.shape[0]
    q = torch.tensor(qkv, dtype=torch.float64, requires_grad=True)
    cf = torch.tensor(cf_seq, dtype=torch.float64)
    G = torch.tensor(dmerged, dtype=torch.float64)
    bias = torch.zeros((N, S, H), dtype=torch.float64, requires_grad=True)  # log cf per head, for cfh
    merged = torch.zeros((T, D), dtype=torch.float64)
    ml = np.zeros((N * H * S, 2))
    ml[:, 0] = -1e30
    outs = []
    for n in range(N):
        cnt = int(off[n + 1] - off[n] + 1)
        rows = torch.tensor([n] + list(range(N + off[n], N + off[n + 1])), dtype=torch.long)
        c = cf[n, :cnt]
        keymask = c > 0
        live = keymask.clone()
        live[0] = True
        logc = torch.where(keymask, torch.log(torch.where(keymask, c, torch.ones_like(c))), torch.zeros_like(c))
        for h in range(H):
            Q = q[rows, h * hd:(h + 1) * hd]
            K = q[rows, D + h * hd:D + (h + 1) * hd]
            V = q[rows, 2 * D + h * hd:2 * D + (h + 1) * hd]
            b = logc + bias[n, :cnt, h]
            s = (Q @ K.T) * sc + b[None, :]
            s = torch.where(keymask[None, :], s, torch.full_like(s, -torch.inf))
            A = torch.softmax(s, dim=1)
            O = (A @ V) * live[:, None].to(torch.float64)
            outs.append((rows, h, O))
            with torch.no_grad():
                m = s.max(dim=1).values
                invl = 1.0 / torch.exp(s - m[:, None]).sum(dim=1)
                for i in range(cnt):
                    if live[i]:
                        ml[(n * H + h) * S + i] = (m[i].item(), invl[i].item())
    loss = 0
    for rows, h, O in outs:
        loss = loss + (O * G[rows, h * hd:(h + 1) * hd]).sum()
        merged[rows, h * hd:(h + 1) * hd] = O.detach()
    loss.backward()
    qkv_adj = q.grad.numpy().copy()
    cfh = bias.grad.numpy().copy()  # [N, S, H]
    with np.errstate(divide="ignore", invalid="ignore"):
        cf_adj = np.where(cf_seq > 0, cfh.sum(axis=2) / np.where(cf_seq > 0, cf_seq, 1.0), 0.0)
    return merged.numpy(), ml, qkv_adj, cfh.reshape(N * S, H), cf_adj


def make(name, counts, H, hd, temperature, cf_kind, extra, seed):
    base = tokens_from_counts(counts, seed=seed, cf_kind=cf_kind)
    S = base.slots + extra
    tk = tokens_from_counts(counts, seed=seed, cf_kind=cf_kind, slots=S)
    rng = np.random.default_rng(100 + seed)
    T = tk.n_rows
    D = H * hd
    qkv = rng.standard_normal((T, 3 * D)).astype(np.float32)
    dmerged = rng.standard_normal((T, D)).astype(np.float32)
    sc = kernel_scale(hd, temperature)
    merged, ml, qkv_adj, cfh, cf_adj = brute_force(qkv, tk.off, tk.cf_seq, dmerged, H, hd, sc)
    path = os.path.join(HERE, f"attn_{name}.npz")
    np.savez_compressed(path, qkv=qkv, off=tk.off, cf_seq=tk.cf_seq, dmerged=dmerged, heads=H, head_dim=hd,
                        temperature=temperature, scale=np.float32(sc), merged=merged, ml=ml, qkv_adj=qkv_adj,
                        cfh=cfh, cf_seq_adj=cf_adj)
    print(f"{path}: N={tk.n_atoms} T={T} S={S} H={H} hd={hd}")


if __name__ == "__main__":
    for name, args in CASES.items():
        make(name, *args)
