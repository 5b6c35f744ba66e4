// pet/forces.hpp -- the consumer of the attention's cf adjoint over the C ABI:
// forces_and_virial for a fixed cutoff (reference peterspackman/pet-kokkos
// src/forces.cpp:345-386) on the reference's PackedEdges arrays
// (include/pet/model.hpp:153-168), fp64 results in caller-owned device memory.
// Errors throw std::runtime_error with the C ABI's message.
#pragma once

#include "attention.hpp"

namespace pet {

// fp64 device views (the reference's RView2D / RView1D).
struct RView2D {
  double* ptr = nullptr;
  int rows = 0, cols = 0;
  double* data() const { return ptr; }
  int extent(int d) const { return d == 0 ? rows : cols; }
};

// An atom-grouped kept-edge list: atom n's edges are off[n] .. off[n+1]-1.
struct PackedEdges {
  int E = 0;                          // rows, dead capacity rows included
  int n_centres = 0;                  // off has n_centres + 1 entries
  const int* off = nullptr;           // [n_centres + 1]
  const int* center = nullptr;        // [E]
  const int* reverse = nullptr;       // [E], -1 if none
  const double* vec = nullptr;        // [E, 3]
  const double* dist = nullptr;       // [E]
  const double* pcut = nullptr;       // [E]
};

enum class CutoffFunction { Bump = 0, Cosine = 1, Smooth = 2 };

// grad [E, 3] = dE/dvec per edge from x4_adj [E, 4], cutoff_adj [E] (may be
// empty) and cf_seq_adj [N, S] (forces_and_virial's "edge_grad" pass).
inline void edge_grad(const PackedEdges& pk, View2D x4_adj, View1D cutoff_adj, View2D cf_seq_adj, double width,
                      CutoffFunction kind, RView2D grad, hipStream_t stream = nullptr) {
  check(pet_edge_grad(pk.n_centres, pk.E, pk.off, pk.center, x4_adj.data(), x4_adj.stride(0), cutoff_adj.data(),
                      cf_seq_adj.data(), cf_seq_adj.stride(0), pk.vec, pk.dist, pk.pcut, width, int(kind),
                      grad.data(), stream),
        "edge_grad");
}

// forces [N, 3] and per-atom virial [N, 9] (fold_edge_gradients, src/forces.cpp:50-68).
inline void fold_edge_gradients(const PackedEdges& pk, int n_atoms, RView2D grad, double scale, RView2D forces,
                                RView2D virial_atom, hipStream_t stream = nullptr) {
  check(pet_fold_edge_gradients(n_atoms, pk.n_centres, pk.off, pk.reverse, pk.vec, grad.data(), scale, forces.data(),
                                virial_atom.data(), stream),
        "fold_edge_gradients");
}

// out [n_struct, width] (= or +=) per-structure sums of x's rows (sum_by_structure, :287-302).
inline void sum_by_structure(RView2D x, const int* soff, RView2D out, bool acc, hipStream_t stream = nullptr) {
  check(pet_sum_by_structure(out.extent(0), x.extent(1), soff, x.data(), out.data(), acc ? 1 : 0, stream),
        "sum_by_structure");
}

// forces_and_virial for a fixed cutoff: forces [N, 3], vir9 [n_struct, 9] and
// edge_grad [E, 3] (fp64, Workspace-owned as the reference's ws.r2 buffers).
inline void forces_and_virial(Workspace& ws, const PackedEdges& pk, int n_atoms, const int* soff, int n_struct,
                              View2D x4_adj, View1D cutoff_adj, View2D cf_seq_adj, double width, CutoffFunction kind,
                              double scale, RView2D& forces, RView2D& vir9, RView2D& grad,
                              hipStream_t stream = nullptr) {
  auto r2 = [&](const std::string& k, int r, int c) {
    return RView2D{static_cast<double*>(ws.bytes(k, sizeof(double) * size_t(r) * size_t(c) + 8)), r, c};
  };
  grad = r2("edge_grad", pk.E, 3);
  forces = r2("forces", n_atoms, 3);
  vir9 = r2("virial9", n_struct, 9);
  const RView2D vir_atom = r2("fold:vir_atom", n_atoms, 9);
  edge_grad(pk, x4_adj, cutoff_adj, cf_seq_adj, width, kind, grad, stream);
  fold_edge_gradients(pk, n_atoms, grad, scale, forces, vir_atom, stream);
  sum_by_structure(vir_atom, soff, vir9, false, stream);
}

}  // namespace pet
