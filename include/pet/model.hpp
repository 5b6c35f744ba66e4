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
//     virial on the host, as the reference's compute() returns them.
// Errors throw std::runtime_error with the C ABI's message.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../pet_model.h"

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
  std::vector<int> off, center, neigh, reverse;
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

// One structure in, energy / forces / virial out (pet::Calculator::compute,
// include/pet/calculator.hpp:187-239), for a fixed-cutoff model. Device
// buffers are kept between calls and grown when a structure needs more.
class Calculator {
 public:
  Calculator(PetModel& model, double cutoff, std::vector<int> species_to_index, hipStream_t stream = nullptr)
      : model_(model), cutoff_(cutoff), s2i_(std::move(species_to_index)), stream_(stream) {}
  Calculator(const Calculator&) = delete;
  Calculator& operator=(const Calculator&) = delete;
  ~Calculator() {
    for (auto& kv : bufs_) (void) hipFree(kv.second.p);
  }

  EnergyResult compute(const System& s, bool forces = true) {
    const auto& h = model_.hypers();
    const HostEdges e = build_edges(s, cutoff_, h.cutoff_width, h.cutoff_function);
    const int N = int(s.positions.size()), E = e.off[N];
    std::vector<int> sp(N), nsp(E), soff{0, N};
    for (int n = 0; n < N; ++n) {
      const int z = s.numbers[n];
      sp[n] = z >= 0 && z < int(s2i_.size()) ? s2i_[z] : -1;
      if (sp[n] < 0) throw std::runtime_error("pet: atomic number " + std::to_string(z) + " not in the model");
    }
    for (int k = 0; k < E; ++k) nsp[k] = sp[e.neigh[k]];
    pet_model_edges d{};
    d.n_atoms = N, d.n_edges = E, d.max_neighbors = e.max_neighbors, d.n_struct = 1;
    d.struct_off = up("soff", soff), d.species = up("sp", sp), d.off = up("off", e.off), d.center = up("c", e.center);
    d.neigh_species = up("nsp", nsp), d.reverse = up("rev", e.reverse), d.vec = up("vec", e.vec);
    d.dist = up("dist", e.dist), d.pcut = up("pcut", e.pcut), d.cut = up("cut", e.cut);
    DeviceOut o;
    o.energy = buf<double>("energy", 1), o.per_atom = buf<double>("per_atom", N);
    if (forces) o.forces = buf<double>("forces", 3 * size_t(N)), o.virial = buf<double>("virial", 9);
    model_.compute(d, forces, o, stream_);
    EnergyResult r;
    r.per_atom.resize(N);
    model_check(hipMemcpyAsync(&r.total, o.energy, sizeof(double), hipMemcpyDeviceToHost, stream_) == hipSuccess
                    ? PET_ATTN_OK
                    : PET_ATTN_ELAUNCH,
                "copy");
    model_check(hipMemcpyAsync(r.per_atom.data(), o.per_atom, sizeof(double) * N, hipMemcpyDeviceToHost, stream_) ==
                        hipSuccess
                    ? PET_ATTN_OK
                    : PET_ATTN_ELAUNCH,
                "copy");
    if (forces) {
      r.forces.resize(3 * size_t(N));
      model_check(hipMemcpyAsync(r.forces.data(), o.forces, sizeof(double) * 3 * N, hipMemcpyDeviceToHost, stream_) ==
                          hipSuccess
                      ? PET_ATTN_OK
                      : PET_ATTN_ELAUNCH,
                  "copy");
      model_check(hipMemcpyAsync(r.virial, o.virial, sizeof(double) * 9, hipMemcpyDeviceToHost, stream_) == hipSuccess
                      ? PET_ATTN_OK
                      : PET_ATTN_ELAUNCH,
                  "copy");
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
  T* up(const std::string& k, const std::vector<T>& v) {
    T* p = buf<T>(k, v.size());
    if (!v.empty())
      model_check(hipMemcpyAsync(p, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice, stream_) == hipSuccess
                      ? PET_ATTN_OK
                      : PET_ATTN_ELAUNCH,
                  "upload");
    return p;
  }

  PetModel& model_;
  double cutoff_;
  std::vector<int> s2i_;
  hipStream_t stream_;
  std::map<std::string, Buf> bufs_;
};

}  // namespace pet
