"""The attention's input side over torch device tensors: the cf_seq bias
source, the token norm and the layer-level attention of a PET block.

``norm_rows`` / ``norm_rows_bwd`` mirror the reference's norm_rows /
norm_rows_bwd (src/ops.hpp:376-436): RMSNorm, or LayerNorm when a bias is
given; ``cf_seq`` its pet_cfseq pass (src/device_neighbors.cpp:318-323);
``attention_layer`` / ``attention_layer_bwd`` the attention block of
PetModel::ff_layer / ff_layer_bwd (src/feedforward.cpp:96-123, :292-329):
tokens -> norm -> qkv = linear(., W_in, b_in) -> attention, and back to the
tokens' adjoint (atom rows set, live edge rows accumulated). All work runs in
libpet_attn.so on the current torch stream.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import Tokens, Workspace, _mat, _ptr, _stream, _weight, shape


def cf_seq(off: torch.Tensor, cut: torch.Tensor, N: int, S: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """cf_seq [N, S]: 1 for the atom's own slot, its kept edges' cutoff factors
    (``cut``, packed order), 0 past its count."""
    lib = _lib.load()
    out = torch.empty((N, S), dtype=torch.float32, device=off.device) if out is None else out
    T = N + (int(cut.numel()) if cut is not None else 0)
    sh = _lib.Shape(N, T, S, 1, 16, 0, 1.0)
    _lib.check(lib.pet_attn_cf_seq(sh, off.data_ptr(), _ptr(cut), out.data_ptr(), _mat(out, "cf_seq", S), _stream()),
               "pet_attn_cf_seq")
    return out


def norm_rows(out: torch.Tensor, inp: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> None:
    """out = norm(inp) row by row (out may be inp)."""
    lib = _lib.load()
    rows, D = inp.shape
    _lib.check(lib.pet_norm_rows(rows, D, out.data_ptr(), _mat(out, "out", D), inp.data_ptr(), _mat(inp, "in", D),
                                 _weight(weight, "weight"), None if bias is None else _weight(bias, "bias"),
                                 _stream()), "pet_norm_rows")


def norm_rows_bwd(in_adj: torch.Tensor, out_adj: torch.Tensor, inp: torch.Tensor, weight: torch.Tensor, ln: bool,
                  beta: float = 0.0) -> None:
    """in_adj = beta * in_adj + the norm's input adjoint for out_adj."""
    lib = _lib.load()
    rows, D = inp.shape
    _lib.check(lib.pet_norm_rows_bwd(rows, D, in_adj.data_ptr(), _mat(in_adj, "in_adj", D), float(beta),
                                     out_adj.data_ptr(), _mat(out_adj, "out_adj", D), inp.data_ptr(),
                                     _mat(inp, "in", D), _weight(weight, "weight"), int(bool(ln)), _stream()),
               "pet_norm_rows_bwd")


def attention_layer(ws: Workspace, key: str, out: torch.Tensor, tokens: torch.Tensor, norm_w: torch.Tensor,
                    norm_b: torch.Tensor | None, w_in: torch.Tensor, b_in: torch.Tensor | None, cf_seq: torch.Tensor,
                    w_out: torch.Tensor, b_out: torch.Tensor | None, tk: Tokens, S: int, heads: int, head_dim: int,
                    temperature: float) -> None:
    """The attention of one PET block from its tokens; the backward's saves
    (merged, ml) stay in ``ws`` under ``key``."""
    lib = _lib.load()
    D = heads * head_dim
    T = tokens.shape[0]
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    merged = ws.n2(key + ":merged", T, D)
    ml = ws.n2(key + ":ml", tk.N * heads * S, 2)
    scratch = ws.bytes("attention_layer:scratch", lib.pet_attention_layer_workspace(sh))
    _lib.check(lib.pet_attention_layer(sh, out.data_ptr(), _mat(out, "out", D), tokens.data_ptr(),
                                       _mat(tokens, "tokens", D), _weight(norm_w, "norm_w"),
                                       None if norm_b is None else _weight(norm_b, "norm_b"), _weight(w_in, "w_in"),
                                       None if b_in is None else _weight(b_in, "b_in"), cf_seq.data_ptr(),
                                       _mat(cf_seq, "cf_seq"), _weight(w_out, "w_out"),
                                       None if b_out is None else _weight(b_out, "b_out"), tk.off.data_ptr(),
                                       merged.data_ptr(), ml.data_ptr(), scratch.data_ptr(), scratch.numel(),
                                       _stream()), "pet_attention_layer")


def attention_layer_bwd(ws: Workspace, key: str, tokens_adj: torch.Tensor, cf_seq_adj: torch.Tensor,
                        out_adj: torch.Tensor, tokens: torch.Tensor, norm_w: torch.Tensor,
                        norm_b: torch.Tensor | None, w_in: torch.Tensor, b_in: torch.Tensor | None,
                        cf_seq: torch.Tensor, w_out: torch.Tensor, tk: Tokens, S: int, heads: int, head_dim: int,
                        temperature: float) -> None:
    """Its backward: tokens_adj's atom rows set, live edge rows accumulated
    (dead rows untouched); cf_seq_adj accumulates."""
    lib = _lib.load()
    D = heads * head_dim
    T = tokens.shape[0]
    sh = shape(tk.N, T, S, heads, head_dim, temperature, tk.dead)
    merged, ml = ws.peek2(key + ":merged"), ws.peek2(key + ":ml")
    scratch = ws.bytes("attention_layer:scratch", lib.pet_attention_layer_workspace(sh))
    _lib.check(lib.pet_attention_layer_bwd(sh, tokens_adj.data_ptr(), _mat(tokens_adj, "tokens_adj", D),
                                           cf_seq_adj.data_ptr(), _mat(cf_seq_adj, "cf_seq_adj"),
                                           out_adj.data_ptr(), _mat(out_adj, "out_adj", D), tokens.data_ptr(),
                                           _mat(tokens, "tokens", D), _weight(norm_w, "norm_w"),
                                           None if norm_b is None else _weight(norm_b, "norm_b"),
                                           _weight(w_in, "w_in"), None if b_in is None else _weight(b_in, "b_in"),
                                           cf_seq.data_ptr(), _mat(cf_seq, "cf_seq"), _weight(w_out, "w_out"),
                                           tk.off.data_ptr(), merged.data_ptr(), ml.data_ptr(), scratch.data_ptr(),
                                           scratch.numel(), _stream()), "pet_attention_layer_bwd")
