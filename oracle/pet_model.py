"""TEST INFRASTRUCTURE ONLY -- the CPU oracle of the whole PET evaluation
(energy, and by autograd the edge gradients that forces and virial fold from).

A restatement in torch (CPU, float64 by default) of the reference's
feedforward- and residual-featurizer passes, written from the weights as the checkpoint stores
them: compress.0 unfolded (the reference folds its constant blocks at load,
src/model.cpp:236-262) and each SwiGLU w_in in metatrain's [value | gate] row
order (the reference interleaves them at load, :211-222). So the fold and the
interleave of the product library are checked, not assumed. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it; the product
has no CPU path.

What each part follows (file:line in the reference tree):
  pass          PetModel::ff_pass            src/feedforward.cpp:338-411
  GNN layer     PetModel::ff_layer           src/feedforward.cpp:34-198
  residual      residual_pass / residual_layer  src/residual.cpp:13-133 (PostLN,
                LayerNorm, SiLU MLP, a readout after every layer, message
                passing input_edge = (input_edge + out_edge(reverse)) / 2)
  compress      compress_fwd + compress.2    src/ops.cpp:326-371, src/feedforward.cpp:64-66
  attention     softmax(sc q.k + log cf)     src/attention.cpp:205-266 (sc :1525)
  norms         norm_rows                    src/ops.hpp:376-407, eps :195-196
  SwiGLU        v * sigmoid(g)               src/ops.cpp:248-279, src/ops.hpp:74-82
  combination   concat / LayerNorm / MLP     src/feedforward.cpp:166-197
  readout       heads and accumulate         src/model.cpp:656-691, src/ops.cpp:406-418
  energy        assemble_energy              src/ops.cpp:420-425
  cutoff        cosine / bump / smooth       include/pet/cutoff.hpp:17-35

Pins (tests/test_oracle_model.py): the attention against the pinned C oracle,
the norms against torch's, edge gradients and forces against central
differences of the energy, permutation and translation invariance, supercell
extensivity, fp32 against fp64; for both featurizers. The model's forward
composition itself (which layer feeds which) has no golden vector here -- the
reference's golden files need published weights that are absent -- so its
parity to the reference is "parity unpinned" beyond these structural checks.
"""
from __future__ import annotations

import math

import numpy as np
import torch

RMS_EPS = 1.1920928955078125e-07  # float32 epsilon (src/ops.hpp:195)
LN_EPS = 1e-5  # (src/ops.hpp:196)


def norm(x, w, b=None):
    """RMSNorm, or LayerNorm when b is given (norm_rows, src/ops.hpp:376-407)."""
    if b is not None:
        mu = x.mean(-1, keepdim=True)
        xc = x - mu
        return xc / torch.sqrt((xc * xc).mean(-1, keepdim=True) + LN_EPS) * w + b
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + RMS_EPS) * w


def linear(x, W, b=None):
    y = x @ W.T
    return y + b if b is not None else y


def silu(x):
    return x * torch.sigmoid(x)


def swiglu(x, w, key):
    """w_out(v * sigmoid(g)), pre = w_in(x) = [v | g] (src/ops.cpp:248-279)."""
    pre = linear(x, w[key + ".w_in.weight"], w[key + ".w_in.bias"])
    F = pre.shape[1] // 2
    return linear(pre[:, :F] * torch.sigmoid(pre[:, F:]), w[key + ".w_out.weight"], w[key + ".w_out.bias"])


def cutoff_factor(d, rc, width, kind):
    """The smooth cutoff factors (include/pet/cutoff.hpp:17-35), differentiable."""
    x = ((d - (rc - width)) / width).clamp(0.0, 1.0)
    if kind == "cosine":
        return 0.5 * (1.0 + torch.cos(math.pi * x))
    if kind == "smooth":
        return 1.0 - x ** 4 * (35.0 - 84.0 * x + 70.0 * x * x - 20.0 * x ** 3)
    # bump: 0.5 (1 + tanh(1 / tan(pi x))) inside (0, 1)
    inside = (x > 0) & (x < 1)
    xs = torch.where(inside, x, torch.full_like(x, 0.5))
    v = 0.5 * (1.0 + torch.tanh(1.0 / torch.tan(math.pi * xs)))
    return torch.where(inside, v, torch.where(x <= 0, torch.ones_like(x), torch.zeros_like(x)))


class TokenIndex:
    """Atom n's tokens: row n, then rows N + off[n] ... (src/ops.hpp:31-37),
    padded to S slots."""

    def __init__(self, off: np.ndarray):
        N = len(off) - 1
        cnt = np.diff(off) + 1
        self.N, self.S = N, int(cnt.max()) if N else 1
        s = np.arange(self.S)[None, :]
        rows = np.where(s == 0, np.arange(N)[:, None], N + off[:-1, None] + s - 1)
        self.valid = torch.from_numpy(s < cnt[:, None])
        self.rows = torch.from_numpy(np.where(s < cnt[:, None], rows, 0).astype(np.int64))
        # edge k's slot: 1 + k - off[center]
        self.cnt = cnt


def attention(qkv, cf_seq, tix: TokenIndex, heads: int, scale: float):
    """merged [T, D]: per (atom, head), softmax over the atom's keys of
    scale q.k + log cf; a query with cf = 0 gives 0 (src/attention.cpp:217-248)."""
    T, D3 = qkv.shape
    D = D3 // 3
    hd = D // heads
    N, S = tix.N, tix.S
    x = qkv[tix.rows.reshape(-1)].reshape(N, S, 3, heads, hd)
    q, k, v = x[:, :, 0].transpose(1, 2), x[:, :, 1].transpose(1, 2), x[:, :, 2].transpose(1, 2)  # [N, H, S, hd]
    live = tix.valid & (cf_seq > 0)  # [N, S]
    logcf = torch.log(torch.where(live, cf_seq, torch.ones_like(cf_seq)))
    s = scale * (q @ k.transpose(-1, -2)) + logcf[:, None, None, :]
    s = s.masked_fill(~live[:, None, None, :], float("-inf"))
    a = torch.softmax(s, dim=-1)
    out = (a @ v).transpose(1, 2)  # [N, S, H, hd]
    out = out * live[:, :, None, None]
    merged = qkv.new_zeros(T, D)
    sel = tix.valid.reshape(-1)
    merged = merged.index_copy(0, tix.rows.reshape(-1)[sel], out.reshape(N * S, D)[sel])
    return merged


def _t(w, dtype):
    return {k: torch.as_tensor(v, dtype=dtype) for k, v in w.items()}


def evaluate(h, weights: dict, species: np.ndarray, pk, composition=None, energy_scale: float = 1.0,
             dtype=torch.float64, grad: bool = True, vec=None):
    """One E(+F) evaluation of a structure (or batch) with packed edges `pk`
    (off, center, neigh, reverse, vec, dist as pet_kokkos_amd.systems.PackedEdges).

    Returns (per_atom energy [N] float64, edge_grad = dE/dvec [E, 3] or None)."""
    w = _t(weights, dtype)
    N = len(species)
    E = int(pk.off[-1])
    D, A, G = h.d_pet, h.num_attention_layers, h.num_gnn_layers
    sp = torch.as_tensor(np.asarray(species), dtype=torch.int64)
    nsp = sp[torch.as_tensor(pk.neigh[:E], dtype=torch.int64)]
    rev = torch.as_tensor(pk.reverse[:E], dtype=torch.int64)
    tix = TokenIndex(np.asarray(pk.off))
    v = torch.tensor(pk.vec[:E], dtype=dtype) if vec is None else vec
    if grad and vec is None:
        v.requires_grad_(True)
    dist = torch.sqrt((v * v).sum(1))
    cut = cutoff_factor(dist, h.cutoff, h.cutoff_width, h.cutoff_function)
    # cf_seq [N, S]: 1, then each edge's factor (src/model.cpp:375-377)
    cf_flat = torch.ones(tix.N * tix.S, dtype=dtype)
    slot = torch.as_tensor(np.arange(E) - pk.off[pk.center[:E]] + 1 + pk.center[:E] * tix.S, dtype=torch.int64)
    cf_flat = cf_flat.index_put((slot,), cut)
    cf_seq = torch.where(tix.valid.reshape(-1), cf_flat, torch.zeros_like(cf_flat)).reshape(tix.N, tix.S)
    x4 = torch.cat([v, dist[:, None]], 1)
    scale = 1.0 / (math.sqrt(h.head_dim) * h.attention_temperature)

    center = torch.as_tensor(pk.center[:E], dtype=torch.int64)

    def head(x, side, i):
        k = f"{side}_heads.energy.{i}"
        y = silu(linear(silu(linear(x, w[k + ".0.weight"], w[k + ".0.bias"])), w[k + ".2.weight"], w[k + ".2.bias"]))
        last = f"{side}_last_layers.energy.{i}.energy___0"
        return linear(y, w[last + ".weight"], w[last + ".bias"])[:, 0]

    def readout(node_feat, edge_feat, i):
        """net of read-out i, in double (readout_accumulate, src/ops.cpp:406-418)."""
        return head(node_feat, "node", i).to(torch.float64).index_add(
            0, center, (cut * head(edge_feat, "edge", i)).to(torch.float64))

    def compress(L, input_edge):
        g = f"gnn_layers.{L}"
        edge_emb = linear(x4, w[g + ".edge_embedder.weight"], w[g + ".edge_embedder.bias"])
        blocks = [edge_emb, input_edge] if L == 0 else [edge_emb, w[g + ".neighbor_embedder.weight"][nsp], input_edge]
        cpre = silu(linear(torch.cat(blocks, 1), w[g + ".compress.0.weight"], w[g + ".compress.0.bias"]))
        return linear(cpre, w[g + ".compress.2.weight"], w[g + ".compress.2.bias"])

    input_edge = w["edge_embedder.weight"][nsp]
    if getattr(h, "residual", False):
        net = torch.zeros(N, dtype=torch.float64)
        for L in range(G):
            g = f"gnn_layers.{L}"
            tokens = torch.cat([w[f"node_embedders.{L}.weight"][sp], compress(L, input_edge)], 0)
            for a in range(A):
                t = f"{g}.trans.layers.{a}"
                qkv = linear(tokens, w[t + ".attention.input_linear.weight"], w[t + ".attention.input_linear.bias"])
                s1 = linear(attention(qkv, cf_seq, tix, h.num_heads, scale), w[t + ".attention.output_linear.weight"],
                            w[t + ".attention.output_linear.bias"]) + tokens
                tok_a = norm(s1, w[t + ".norm_attention.weight"], w[t + ".norm_attention.bias"])
                hmid = silu(linear(tok_a, w[t + ".mlp.w_in.weight"], w[t + ".mlp.w_in.bias"]))
                s2 = linear(hmid, w[t + ".mlp.w_out.weight"], w[t + ".mlp.w_out.bias"]) + tok_a
                tokens = norm(s2, w[t + ".norm_mlp.weight"], w[t + ".norm_mlp.bias"])
            net = net + readout(tokens[:N], tokens[N:], L)
            if L + 1 < G:
                back = torch.where((rev >= 0)[:, None], tokens[N:][rev.clamp(min=0)], torch.zeros_like(tokens[N:]))
                input_edge = 0.5 * (input_edge + back)
        return _finish(net, sp, h, composition, energy_scale, grad, v)

    node = w["node_embedders.0.weight"][sp]
    for L in range(G):
        g = f"gnn_layers.{L}"
        edge_cur = compress(L, input_edge)
        node_cur = node
        for a in range(A):
            t = f"{g}.trans.layers.{a}"
            input_node = linear(node_cur, w[t + ".center_contraction.weight"], w[t + ".center_contraction.bias"])
            tokens = torch.cat([input_node, edge_cur], 0)
            qkv = linear(norm(tokens, w[t + ".norm_attention.weight"]), w[t + ".attention.input_linear.weight"],
                         w[t + ".attention.input_linear.bias"])
            attn = linear(attention(qkv, cf_seq, tix, h.num_heads, scale), w[t + ".attention.output_linear.weight"],
                          w[t + ".attention.output_linear.bias"])
            node_res = node_cur + linear(attn[:N], w[t + ".center_expansion.weight"], w[t + ".center_expansion.bias"])
            eps = attn[N:] + edge_cur
            node_cur = node_res + swiglu(norm(node_res, w[t + ".norm_center_features.weight"]), w, t + ".center_mlp")
            edge_cur = eps + swiglu(norm(eps, w[t + ".norm_mlp.weight"]), w, t + ".mlp")
        node = node_cur
        back = torch.where((rev >= 0)[:, None], edge_cur[rev.clamp(min=0)], torch.zeros_like(edge_cur))
        cat = torch.cat([edge_cur, back], 1)
        cn = norm(cat, w[f"combination_norms.{L}.weight"], w[f"combination_norms.{L}.bias"])
        comb = linear(silu(linear(cn, w[f"combination_mlps.{L}.0.weight"], w[f"combination_mlps.{L}.0.bias"])),
                      w[f"combination_mlps.{L}.2.weight"], w[f"combination_mlps.{L}.2.bias"])
        input_edge = input_edge + edge_cur + comb

    return _finish(readout(node, input_edge, 0), sp, h, composition, energy_scale, grad, v)


def _finish(net, sp, h, composition, energy_scale, grad, v):
    comp = torch.zeros(h.n_species, dtype=torch.float64) if composition is None else \
        torch.as_tensor(composition, dtype=torch.float64)
    per_atom = energy_scale * net + comp[sp]
    eg = None
    if grad:
        (eg,) = torch.autograd.grad(per_atom.sum(), v)
        eg = eg.detach().to(torch.float64).numpy()
    return per_atom.detach().numpy(), eg


def fold_forces(n_atoms: int, pk, edge_grad: np.ndarray, scale: float = 1.0):
    """forces [N, 3] and per-atom virial [N, 9] from dE/dvec, by the fold of
    src/forces.cpp:50-68 (vectorised: F_i = -sum_{k: j(k)=i}... as the
    reference's partner form, which equals the centre/neighbour scatter)."""
    E = int(pk.off[-1])
    g = edge_grad[:E]
    f = np.zeros((n_atoms, 3))
    # v_k = r_j - r_i: dE/dr_i -= g_k, dE/dr_j += g_k; forces = -dE/dr
    np.add.at(f, pk.center[:E], g)
    np.add.at(f, pk.neigh[:E], -g)
    vir = np.zeros((n_atoms, 9))
    np.add.at(vir, pk.center[:E], (pk.vec[:E, :, None] * g[:, None, :]).reshape(E, 9))
    return scale * f, scale * vir
