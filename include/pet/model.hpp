// pet/model.hpp -- the reference's PetModel and Calculator over the C ABI of
// pet_model.h, for a C++ caller (peterspackman/pet-kokkos include/pet/model.hpp,
// include/pet/calculator.hpp:187-239, src/neighbors.cpp:176-260):
//   - PetModel takes the checkpoint's tensors by name (the reference's
//     Checkpoint::weights, include/pet/safetensors.hpp) and evaluates packed
//     edges already on the device (DeviceEdgeData + PackedEdges);
//   - build_edges is a host neighbour list of a periodic structure in the
//     reference's raw-edge order (every (i, j, image) with 0 < |v| <= cutoff,
//     grouped by centre, images in increasing shift order), with each edge's
//     reverse and its cosine or bump cutoff factor;
//   - Calculator::compute runs both for one structure: energy, forces and
//     virial on the host, as the reference's compute() returns them; its
//     set_neighbors / compute_step / compute_edges keep an MD engine's list on
//     the device between steps.
// Errors throw std::runtime_error with the C ABI's message.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../pet_model.h"
#include "replay.hpp"

namespace pet {

// One checkpoint tensor: row-major float64 (include/pet/safetensors.hpp).
struct Tensor {
  std::vector<int64_t> shape;
  std::vector<double> data;
};

inline void model_check(int code, const char* what) {
  if (code != PET_ATTN_OK) throw std::runtime_error(std::string("pet: ") + what + ": " + pet_attn_strerror(code));
}

// Device outputs of one evaluation (fp64): any may be null but forces, which
// a forces run needs.
struct DeviceOut {
  double* energy = nullptr;    // [B]
  double* per_atom = nullptr;  // [N]
  double* forces = nullptr;    // [N, 3]
  double* virial = nullptr;    // [B, 9]
  double* edge_grad = nullptr; // [E, 3]
};

class PetModel {
 public:
  PetModel(const pet_model_hypers& h, const std::map<std::string, Tensor>& weights,
           const std::vector<double>& composition)
      : h_(h) {
    std::vector<pet_model_tensor> t;
    t.reserve(weights.size());
    for (const auto& [name, ten] : weights) {
      if (ten.shape.empty() || ten.shape.size() > 2) throw std::runtime_error("pet: tensor '" + name + "' not 1D/2D");
      t.push_back({name.c_str(), int(ten.shape[0]), ten.shape.size() == 2 ? int(ten.shape[1]) : 0, ten.data.data()});
    }
    model_check(pet_model_create(&h, t.data(), int(t.size()), composition.empty() ? nullptr : composition.data(), &m_),
                "PetModel");
  }
  PetModel(const PetModel&) = delete;
  PetModel& operator=(const PetModel&) = delete;
  ~PetModel() { pet_model_destroy(m_); }

  const pet_model_hypers& hypers() const { return h_; }
  size_t workspace_bytes() const { return pet_model_workspace_bytes(m_); }
  size_t pairs_scratch_bytes() const { return pet_model_pairs_scratch_bytes(m_); }
  int last_tier() const { return pet_model_last_tier(m_); }

  // energy_forces_batch on the device (src/model.cpp:795-811).
  void compute(const pet_model_edges& edges, bool forces, const DeviceOut& out, hipStream_t stream = nullptr) {
    model_check(pet_model_compute(m_, &edges, forces ? 1 : 0, out.energy, out.per_atom, out.forces, out.virial,
                                  out.edge_grad, stream),
                "PetModel::compute");
  }

 private:
  pet_model_hypers h_;
  pet_model* m_ = nullptr;
};

// A periodic structure (include/pet/calculator.hpp's System).
struct System {
  std::vector<std::array<double, 3>> positions;
  std::array<std::array<double, 3>, 3> cell;  // rows are lattice vectors
  std::vector<int> numbers;
};

// A host neighbour list, packed: atom n's edges off[n] .. off[n+1]-1.
struct HostEdges {
  std::vector<int> off, center, neigh, reverse, shift;  // shift [E, 3]
  std::vector<double> vec, dist, pcut;  // [E, 3], [E], [E]
  std::vector<float> cut;
  int max_neighbors = 0;
};

// The smooth cutoff factor (include/pet/cutoff.hpp:17-35): 0 bump, 1 cosine.
inline double cutoff_factor(double d, double rc, double w, int kind) {
  const double x = (d - (rc - w)) / w;
  if (x <= 0.0) return 1.0;
  if (x >= 1.0) return 0.0;
  const double pi = 3.14159265358979323846;
  if (kind == 1) return 0.5 * (1.0 + std::cos(pi * x));
  if (kind == 0) return 0.5 * (1.0 + std::tanh(1.0 / std::tan(pi * x)));
  const double x4 = x * x * x * x;
  return 1.0 - x4 * (35.0 - 84.0 * x + 70.0 * x * x - 20.0 * x * x * x);
}

// Every (i, j, image) with 0 < |r_j + shift - r_i| <= cutoff, centre-major, then
// j, then the image shifts in increasing order (src/neighbors.cpp:176-247).
inline HostEdges build_edges(const System& s, double cutoff, double width, int kind) {
  const int N = int(s.positions.size());
  const auto& a = s.cell;
  // images needed along each lattice vector: cutoff over the distance between
  // the two faces the other vectors span
  auto cross = [](const std::array<double, 3>& u, const std::array<double, 3>& v) {
    return std::array<double, 3>{u[1] * v[2] - u[2] * v[1], u[2] * v[0] - u[0] * v[2], u[0] * v[1] - u[1] * v[0]};
  };
  auto dot = [](const std::array<double, 3>& u, const std::array<double, 3>& v) {
    return u[0] * v[0] + u[1] * v[1] + u[2] * v[2];
  };
  const double vol = std::fabs(dot(a[0], cross(a[1], a[2])));
  int rng[3];
  for (int k = 0; k < 3; ++k) {
    const auto c = cross(a[(k + 1) % 3], a[(k + 2) % 3]);
    rng[k] = int(std::ceil(cutoff / (vol / std::sqrt(dot(c, c)))));
  }
  struct Key {
    int i, j, x, y, z;
    bool operator==(const Key& o) const { return i == o.i && j == o.j && x == o.x && y == o.y && z == o.z; }
  };
  struct Hash {
    size_t operator()(const Key& k) const {
      return (size_t(k.i) * 1000003u) ^ (size_t(k.j) * 19349663u) ^ (size_t(k.x + 64) * 83492791u) ^
             (size_t(k.y + 64) * 2654435761u) ^ size_t(k.z + 64);
    }
  };
  HostEdges e;
  std::vector<Key> keys;
  std::unordered_map<Key, int, Hash> index;
  e.off.assign(N + 1, 0);
  const double c2 = cutoff * cutoff;
  for (int i = 0; i < N; ++i) {
    e.off[i] = int(e.center.size());
    for (int j = 0; j < N; ++j)
      for (int x = -rng[0]; x <= rng[0]; ++x)
        for (int y = -rng[1]; y <= rng[1]; ++y)
          for (int z = -rng[2]; z <= rng[2]; ++z) {
            double v[3];
            for (int c = 0; c < 3; ++c)
              v[c] = s.positions[j][c] + x * a[0][c] + y * a[1][c] + z * a[2][c] - s.positions[i][c];
            const double d2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
            if (d2 < 1e-24 || d2 > c2) continue;
            const double d = std::sqrt(d2);
            index[Key{i, j, x, y, z}] = int(e.center.size());
            keys.push_back(Key{i, j, x, y, z});
            e.center.push_back(i), e.neigh.push_back(j);
            e.shift.insert(e.shift.end(), {x, y, z});
            e.vec.insert(e.vec.end(), v, v + 3);
            e.dist.push_back(d), e.pcut.push_back(cutoff);
            e.cut.push_back(float(cutoff_factor(d, cutoff, width, kind)));
          }
    e.max_neighbors = std::max(e.max_neighbors, int(e.center.size()) - e.off[i]);
  }
  e.off[N] = int(e.center.size());
  e.reverse.resize(keys.size());
  for (size_t k = 0; k < keys.size(); ++k) {
    auto it = index.find(Key{keys[k].j, keys[k].i, -keys[k].x, -keys[k].y, -keys[k].z});
    e.reverse[k] = it == index.end() ? -1 : it->second;
  }
  return e;
}

struct EnergyResult {
  double total = 0.0;
  std::vector<double> per_atom;  // [N] eV
  std::vector<double> forces;    // [N, 3] eV/A
  double virial[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};  // sum v (x) dE/dv, row-major 3x3, eV
};

// An MD engine's full neighbour list (the reference's EdgeListView,
// include/pet/device_geometry.hpp:93-110): atom i's neighbours are
// neighbors[offsets[i] .. offsets[i+1]-1], each with an optional lattice shift
// (cell rows); every atom is a centre and owned.
struct EdgeListView {
  int n_atoms = 0;
  const double* positions = nullptr;  // [n_atoms, 3] A
  const int* atomic_numbers = nullptr;
  const int* offsets = nullptr;       // [n_atoms + 1]
  const int* neighbors = nullptr;     // [offsets[n_atoms]]
  const int* shifts = nullptr;        // [offsets[n_atoms], 3], optional
  const double* cell = nullptr;       // [9], with shifts
};

// One structure in, energy / forces / virial out (pet::Calculator,
// include/pet/calculator.hpp:187-239), for a fixed-cutoff model. compute()
// builds the neighbour list on the host; set_neighbors() + compute_step() keep
// an engine's list on the device and move only positions each step (pairs that
// drift past the cutoff weigh nothing); compute_edges() is both at once. Edge
// geometry is always made on the device (pet_edge_geometry). Device buffers
// are kept between calls and grown when a structure needs more.
//
// With graph = true (and a non-null stream: capture needs one; on the null
// stream the steps stay eager), compute_step replays its device work -- edge
// geometry and the whole evaluation -- as one HIP graph per output set from the
// second step on a list (pet::StepRecorder): positions are copied into the buffer
// the graph reads, the results are the bits of an eager step, and a small
// structure's step loses most of its launch cost. set_neighbors drops the
// recorded graphs.
class Calculator {
 public:
  Calculator(PetModel& model, double cutoff, std::vector<int> species_to_index, hipStream_t stream = nullptr,
             bool graph = false)
      : model_(model), cutoff_(cutoff), s2i_(std::move(species_to_index)), stream_(stream) {
    if (graph) graphs_ = std::make_unique<StepRecorder>(stream);
  }
  Calculator(const Calculator&) = delete;
  Calculator& operator=(const Calculator&) = delete;
  ~Calculator() {
    for (auto& kv : bufs_) (void) hipFree(kv.second.p);
  }

  EnergyResult compute(const System& s, bool forces = true) {
    const auto& h = model_.hypers();
    const HostEdges e = build_edges(s, cutoff_, h.cutoff_width, h.cutoff_function);
    const int N = int(s.positions.size());
    std::vector<int> z(s.numbers), nb(e.neigh);
    std::vector<double> pos(3 * size_t(N)), cell(9);
    for (int n = 0; n < N; ++n)
      for (int c = 0; c < 3; ++c) pos[3 * size_t(n) + c] = s.positions[n][c];
    for (int r = 0; r < 3; ++r)
      for (int c = 0; c < 3; ++c) cell[3 * r + c] = s.cell[r][c];
    EdgeListView v;
    v.n_atoms = N, v.positions = pos.data(), v.atomic_numbers = z.data(), v.offsets = e.off.data();
    v.neighbors = nb.data(), v.shifts = e.shift.data(), v.cell = cell.data();
    return compute_edges(v, forces);
  }

  // set_neighbors then compute_step (Calculator::compute_edges, include/pet/calculator.hpp:219-227).
  EnergyResult compute_edges(const EdgeListView& v, bool forces = true, std::vector<double>* edge_gradient = nullptr) {
    set_neighbors(v);
    return compute_step(v.positions, v.cell, forces, edge_gradient);
  }

  // The list's topology to the device, once per rebuild (Calculator::set_neighbors).
  void set_neighbors(const EdgeListView& v) {
    const int N = v.n_atoms;
    if (N < 0 || (N > 0 && (!v.atomic_numbers || !v.offsets))) throw std::runtime_error("pet: bad neighbour list");
    const int E = N ? v.offsets[N] : 0;
    if (E > 0 && !v.neighbors) throw std::runtime_error("pet: bad neighbour list");
    std::vector<int> sp(N), nsp(E), center(E), rev(E, -1);
    int maxc = 0;
    for (int n = 0; n < N; ++n) {
      const int z = v.atomic_numbers[n];
      sp[n] = z >= 0 && z < int(s2i_.size()) ? s2i_[z] : -1;
      if (sp[n] < 0) throw std::runtime_error("pet: atomic number " + std::to_string(z) + " not in the model");
      if (v.offsets[n + 1] < v.offsets[n]) throw std::runtime_error("pet: offsets not increasing");
      maxc = std::max(maxc, v.offsets[n + 1] - v.offsets[n]);
      for (int k = v.offsets[n]; k < v.offsets[n + 1]; ++k) center[k] = n;
    }
    // each edge's reverse (j, i, -shift), by a hash of (i, j, shift)
    struct Hash {
      size_t operator()(const std::array<int, 5>& k) const {
        size_t x = 1469598103934665603ull;
        for (int t : k) x = (x ^ size_t(uint32_t(t))) * 1099511628211ull;
        return x;
      }
    };
    std::unordered_map<std::array<int, 5>, int, Hash> index;
    auto key = [&](int k, int sign) {
      const int* sh = v.shifts ? v.shifts + 3 * size_t(k) : nullptr;
      return sign > 0 ? std::array<int, 5>{center[k], v.neighbors[k], sh ? sh[0] : 0, sh ? sh[1] : 0, sh ? sh[2] : 0}
                      : std::array<int, 5>{v.neighbors[k], center[k], sh ? -sh[0] : 0, sh ? -sh[1] : 0,
                                           sh ? -sh[2] : 0};
    };
    for (int k = 0; k < E; ++k) {
      if (v.neighbors[k] < 0 || v.neighbors[k] >= N) throw std::runtime_error("pet: neighbour index out of range");
      nsp[k] = sp[v.neighbors[k]];
      index[key(k, 1)] = k;
    }
    for (int k = 0; k < E; ++k) {
      auto it = index.find(key(k, -1));
      rev[k] = it == index.end() ? -1 : it->second;
    }
    std::vector<int> soff{0, N}, off(v.offsets, v.offsets + N + 1), nb(v.neighbors, v.neighbors + E);
    std::vector<int> sh(v.shifts ? v.shifts : nullptr, v.shifts ? v.shifts + 3 * size_t(E) : nullptr);
    d_ = pet_model_edges{};
    d_.n_atoms = N, d_.n_edges = E, d_.max_neighbors = maxc, d_.n_struct = 1;
    d_.struct_off = up("soff", soff), d_.species = up("sp", sp), d_.off = up("off", off), d_.center = up("c", center);
    d_.neigh_species = up("nsp", nsp), d_.reverse = up("rev", rev);
    neigh_ = up("nb", nb), shift_ = v.shifts ? up("sh", sh) : nullptr;
    d_.vec = buf<double>("vec", 3 * size_t(E)), d_.dist = buf<double>("dist", E), d_.pcut = buf<double>("pcut", E);
    d_.cut = buf<float>("cut", E);
    model_check(hipStreamSynchronize(stream_) == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH, "synchronize");
    if (graphs_) graphs_->forget();
    have_list_ = true;
  }

  // Whether a step's capture failed (that output set then runs eagerly).
  bool graph_broken() const { return graphs_ && graphs_->counters().refusals > 0; }
  // The recorder's counters (all zero without graph = true).
  StepRecorder::Counters graph_counters() const { return graphs_ ? graphs_->counters() : StepRecorder::Counters{}; }

  // One step on the list set_neighbors holds, with the atoms' positions in its
  // order (Calculator::compute_step, include/pet/calculator.hpp:228-230).
  EnergyResult compute_step(const double* positions, const double* cell = nullptr, bool forces = true,
                            std::vector<double>* edge_gradient = nullptr) {
    if (!have_list_) throw std::runtime_error("pet: compute_step before set_neighbors");
    if (shift_ && !cell) throw std::runtime_error("pet: the list has shifts, so compute_step needs the cell");
    const auto& h = model_.hypers();
    const int N = d_.n_atoms, E = d_.n_edges;
    double* pos = buf<double>("pos", 3 * size_t(N));
    double* dcell = buf<double>("cell", 9);
    DeviceOut o;
    o.energy = buf<double>("energy", 1), o.per_atom = buf<double>("per_atom", N);
    if (forces) o.forces = buf<double>("forces", 3 * size_t(N)), o.virial = buf<double>("virial", 9);
    if (forces && edge_gradient) o.edge_grad = buf<double>("edge_grad", 3 * size_t(E));
    copy_in(pos, positions, 3 * size_t(N));
    if (cell) copy_in(dcell, cell, 9);
    auto work = [&] {
      model_check(pet_edge_geometry(E, d_.center, neigh_, shift_, pos, shift_ ? dcell : nullptr, cutoff_,
                                    h.cutoff_width, h.cutoff_function, const_cast<double*>(d_.vec),
                                    const_cast<double*>(d_.dist), const_cast<double*>(d_.pcut),
                                    const_cast<float*>(d_.cut), stream_),
                  "edge geometry");
      model_.compute(d_, forces, o, stream_);
    };
    if (graphs_) {
      // every buffer the recorded work reads or writes, by address
      Signature sig{std::uint64_t(forces)};
      sig.add(pos).add(dcell).add(o.energy).add(o.per_atom).add(o.forces).add(o.virial).add(o.edge_grad).add(d_.vec);
      graphs_->launch(sig, work);
    } else {
      work();
    }
    EnergyResult r;
    r.per_atom.resize(N);
    copy_out(&r.total, o.energy, 1);
    copy_out(r.per_atom.data(), o.per_atom, N);
    if (forces) {
      r.forces.resize(3 * size_t(N));
      copy_out(r.forces.data(), o.forces, 3 * size_t(N));
      copy_out(r.virial, o.virial, 9);
      if (edge_gradient) {
        edge_gradient->resize(3 * size_t(E));
        copy_out(edge_gradient->data(), o.edge_grad, 3 * size_t(E));
      }
    }
    model_check(hipStreamSynchronize(stream_) == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH, "synchronize");
    return r;
  }

 private:
  struct Buf {
    void* p = nullptr;
    size_t size = 0;
  };
  template <class T>
  T* buf(const std::string& k, size_t n) {
    Buf& b = bufs_[k];
    const size_t need = sizeof(T) * (n ? n : 1);
    if (b.size < need) {
      model_check(hipStreamSynchronize(stream_) == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH, "synchronize");
      if (b.p) (void) hipFree(b.p);
      b.p = nullptr, b.size = 0;
      if (hipMalloc(&b.p, need) != hipSuccess) throw std::runtime_error("pet: device allocation failed");
      b.size = need;
    }
    return static_cast<T*>(b.p);
  }
  template <class T>
  void copy_in(T* dst, const T* src, size_t n) {
    if (n)
      model_check(hipMemcpyAsync(dst, src, sizeof(T) * n, hipMemcpyHostToDevice, stream_) == hipSuccess
                      ? PET_ATTN_OK
                      : PET_ATTN_ELAUNCH,
                  "upload");
  }
  template <class T>
  void copy_out(T* dst, const T* src, size_t n) {
    if (n)
      model_check(hipMemcpyAsync(dst, src, sizeof(T) * n, hipMemcpyDeviceToHost, stream_) == hipSuccess
                      ? PET_ATTN_OK
                      : PET_ATTN_ELAUNCH,
                  "download");
  }
  template <class T>
  T* up(const std::string& k, const std::vector<T>& v) {
    T* p = buf<T>(k, v.size());
    copy_in(p, v.data(), v.size());
    return p;
  }

  PetModel& model_;
  double cutoff_;
  std::vector<int> s2i_;
  hipStream_t stream_;
  std::map<std::string, Buf> bufs_;
  pet_model_edges d_{};
  const int* neigh_ = nullptr;
  const int* shift_ = nullptr;
  bool have_list_ = false;
  std::unique_ptr<StepRecorder> graphs_;
};

}  // namespace pet
