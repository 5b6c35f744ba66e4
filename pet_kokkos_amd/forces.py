"""The consumer of the attention's cf adjoint over torch device tensors:
forces_and_virial's edge term, the fold of edge gradients into forces and
per-atom virials, and the sum over structures (reference src/forces.cpp:50-70,
:287-302, :345-378; the adaptive cutoff's share is not part of this path).
All work runs in libpet_attn.so on the current torch stream.
"""
from __future__ import annotations

import dataclasses

import torch

from . import _lib
from .attention import _mat, _ptr, _stream

CUTOFF_KINDS = {"bump": 0, "cosine": 1, "smooth": 2}


@dataclasses.dataclass
class PackedEdges:
    """Device copy of an atom-grouped edge list (include/pet/model.hpp:153-168)."""
    off: torch.Tensor  # int32 [n_centres + 1]
    center: torch.Tensor  # int32 [E]
    reverse: torch.Tensor  # int32 [E], -1 if none
    vec: torch.Tensor  # float64 [E, 3]
    dist: torch.Tensor  # float64 [E]
    pcut: torch.Tensor  # float64 [E]

    @staticmethod
    def from_host(pk, device) -> "PackedEdges":
        def t(a, dt):
            return torch.as_tensor(a, dtype=dt).to(device).contiguous()
        return PackedEdges(t(pk.off, torch.int32), t(pk.center, torch.int32), t(pk.reverse, torch.int32),
                           t(pk.vec, torch.float64), t(pk.dist, torch.float64), t(pk.pcut, torch.float64))

    @property
    def n_edges(self) -> int:
        return int(self.center.numel())

    @property
    def n_centres(self) -> int:
        return int(self.off.numel()) - 1


def _f64(t: torch.Tensor, name: str, n: int) -> int:
    if t.device.type != "cuda" or t.dtype != torch.float64 or not t.is_contiguous() or t.numel() != n:
        raise ValueError(f"{name} must be a contiguous float64 device tensor of {n} elements")
    return t.data_ptr()


def edge_grad(pk: PackedEdges, x4_adj: torch.Tensor, cutoff_adj: torch.Tensor | None, cf_seq_adj: torch.Tensor,
              width: float, kind: int | str, grad: torch.Tensor | None = None) -> torch.Tensor:
    """grad [E, 3] fp64 = dE/dvec per edge from the readout's (vec, |vec|)
    adjoint x4_adj [E, 4], the cutoff adjoints and the attention's cf_seq_adj."""
    lib = _lib.load()
    kind = CUTOFF_KINDS[kind] if isinstance(kind, str) else int(kind)
    E = pk.n_edges
    grad = torch.empty((E, 3), dtype=torch.float64, device=pk.vec.device) if grad is None else grad
    if cutoff_adj is not None and (cutoff_adj.dtype != torch.float32 or not cutoff_adj.is_contiguous()):
        raise ValueError("cutoff_adj must be a contiguous float32 tensor")
    _lib.check(lib.pet_edge_grad(pk.n_centres, E, pk.off.data_ptr(), pk.center.data_ptr(), x4_adj.data_ptr(),
                                 _mat(x4_adj, "x4_adj", 4), _ptr(cutoff_adj), cf_seq_adj.data_ptr(),
                                 _mat(cf_seq_adj, "cf_seq_adj"), _f64(pk.vec, "vec", 3 * E),
                                 _f64(pk.dist, "dist", E), _f64(pk.pcut, "pcut", E), float(width), kind,
                                 _f64(grad, "grad", 3 * E), _stream()), "pet_edge_grad")
    return grad


def fold_edge_gradients(pk: PackedEdges, n_atoms: int, grad: torch.Tensor, scale: float = 1.0):
    """(forces [N, 3], per-atom virial [N, 9]), fp64."""
    lib = _lib.load()
    dev = grad.device
    forces = torch.empty((n_atoms, 3), dtype=torch.float64, device=dev)
    vir = torch.empty((n_atoms, 9), dtype=torch.float64, device=dev)
    _lib.check(lib.pet_fold_edge_gradients(n_atoms, pk.n_centres, pk.off.data_ptr(), pk.reverse.data_ptr(),
                                           _f64(pk.vec, "vec", 3 * pk.n_edges), _f64(grad, "grad", 3 * pk.n_edges),
                                           float(scale), forces.data_ptr(), vir.data_ptr(), _stream()),
               "pet_fold_edge_gradients")
    return forces, vir


def sum_by_structure(soff: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None,
                     accumulate: bool = False) -> torch.Tensor:
    """Per-structure sums [n_struct, width] of x's rows, atoms soff[b] .. soff[b+1]-1."""
    lib = _lib.load()
    NS, W = int(soff.numel()) - 1, int(x.shape[1])
    out = torch.zeros((NS, W), dtype=torch.float64, device=x.device) if out is None else out
    _lib.check(lib.pet_sum_by_structure(NS, W, soff.data_ptr(), _f64(x, "x", x.numel()), _f64(out, "out", NS * W),
                                        int(accumulate), _stream()), "pet_sum_by_structure")
    return out


def forces_and_virial(pk: PackedEdges, n_atoms: int, soff: torch.Tensor, x4_adj: torch.Tensor,
                      cutoff_adj: torch.Tensor | None, cf_seq_adj: torch.Tensor, width: float, kind: int | str,
                      scale: float = 1.0):
    """(forces [N, 3], virial [n_struct, 9], edge grad [E, 3]) of the reference's
    forces_and_virial for a fixed cutoff (src/forces.cpp:345-386)."""
    grad = edge_grad(pk, x4_adj, cutoff_adj, cf_seq_adj, width, kind)
    forces, vir_atom = fold_edge_gradients(pk, n_atoms, grad, scale)
    return forces, sum_by_structure(soff, vir_atom), grad
