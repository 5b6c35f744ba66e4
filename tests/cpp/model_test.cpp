// Drives the whole PET evaluation through the C++ interface
// (include/pet/model.hpp: PetModel, build_edges, Calculator) as a C++ caller
// of the reference's would, for tests/test_gpu_cpp_api.py:
//
//   model_test DIR
//
// reads DIR/hypers.txt (d_pet d_node d_head heads gnn_layers attention_layers
// n_species cutoff_function cutoff_width temperature energy_scale cutoff featurizer),
// DIR/manifest.txt ("name rows cols" a tensor, cols 0 for a vector) with
// DIR/weights.f64 (the tensors back to back), DIR/composition.f64,
// DIR/s2i.txt (species_to_index) and DIR/system.txt (N, the cell's 9 numbers,
// then "Z x y z" an atom). Writes DIR/result.f64 = [energy, per_atom (N),
// forces (3N), virial (9)], DIR/repeat.ok when a second evaluation gives the
// same bits, and DIR/fd.f64 = [central difference of the energy in atom 0's x
// (step 1e-3 A, energy-only runs), the force's x], and DIR/graph.ok when
// compute_step on a Calculator with graph = true (a stream of its own) gives
// the bits of an eager Calculator's on the same list, step after step, with
// and without forces and edge gradients, and DIR/linear.ok when
// pet::linear_fused (include/pet/linear.hpp) on plain and on split weights
// agrees with a host double product within 1e-5 of its largest magnitude.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "pet/linear.hpp"
#include "pet/model.hpp"

static void fail(const std::string& what) {
  std::fprintf(stderr, "model_test: %s\n", what.c_str());
  std::exit(2);
}

int main(int argc, char** argv) {
  if (argc != 2) fail("usage: model_test DIR");
  const std::string dir = argv[1];
  std::ifstream hf(dir + "/hypers.txt");
  pet_model_hypers h{};
  double cutoff = 0;
  if (!(hf >> h.d_pet >> h.d_node >> h.d_head >> h.num_heads >> h.num_gnn_layers >> h.num_attention_layers >>
        h.n_species >> h.cutoff_function >> h.cutoff_width >> h.attention_temperature >> h.energy_scale >> cutoff >>
        h.featurizer))
    fail("hypers.txt");
  std::ifstream mf(dir + "/manifest.txt");
  FILE* wf = std::fopen((dir + "/weights.f64").c_str(), "rb");
  if (!wf) fail("weights.f64");
  std::map<std::string, pet::Tensor> w;
  std::string name;
  int rows = 0, cols = 0;
  while (mf >> name >> rows >> cols) {
    pet::Tensor t;
    t.shape = cols ? std::vector<int64_t>{rows, cols} : std::vector<int64_t>{rows};
    t.data.resize(size_t(rows) * (cols ? cols : 1));
    if (std::fread(t.data.data(), sizeof(double), t.data.size(), wf) != t.data.size()) fail("weights.f64 short");
    w[name] = std::move(t);
  }
  std::fclose(wf);
  std::vector<double> comp(h.n_species);
  FILE* cf = std::fopen((dir + "/composition.f64").c_str(), "rb");
  if (!cf || std::fread(comp.data(), sizeof(double), comp.size(), cf) != comp.size()) fail("composition.f64");
  std::fclose(cf);
  std::ifstream sf(dir + "/s2i.txt");
  std::vector<int> s2i;
  for (int v; sf >> v;) s2i.push_back(v);
  std::ifstream yf(dir + "/system.txt");
  pet::System s;
  int N = 0;
  yf >> N;
  for (auto& r : s.cell)
    for (double& c : r) yf >> c;
  s.positions.resize(N), s.numbers.resize(N);
  for (int n = 0; n < N; ++n) yf >> s.numbers[n] >> s.positions[n][0] >> s.positions[n][1] >> s.positions[n][2];
  if (!yf) fail("system.txt");

  try {
    pet::PetModel model(h, w, comp);
    pet::Calculator calc(model, cutoff, s2i);
    const pet::EnergyResult r = calc.compute(s, true);
    std::vector<double> out{r.total};
    out.insert(out.end(), r.per_atom.begin(), r.per_atom.end());
    out.insert(out.end(), r.forces.begin(), r.forces.end());
    out.insert(out.end(), r.virial, r.virial + 9);
    FILE* of = std::fopen((dir + "/result.f64").c_str(), "wb");
    std::fwrite(out.data(), sizeof(double), out.size(), of);
    std::fclose(of);

    const pet::EnergyResult r2 = calc.compute(s, true);
    if (r2.total == r.total && std::memcmp(r2.forces.data(), r.forces.data(), sizeof(double) * r.forces.size()) == 0 &&
        std::memcmp(r2.virial, r.virial, sizeof r.virial) == 0)
      std::fclose(std::fopen((dir + "/repeat.ok").c_str(), "wb"));

    const double step = 1e-3;
    pet::System sp = s, sm = s;
    sp.positions[0][0] += step, sm.positions[0][0] -= step;
    const double ep = calc.compute(sp, false).total, em = calc.compute(sm, false).total;
    const double fd[2] = {-(ep - em) / (2 * step), r.forces[0]};
    FILE* ff = std::fopen((dir + "/fd.f64").c_str(), "wb");
    std::fwrite(fd, sizeof(double), 2, ff);
    std::fclose(ff);

    hipStream_t st = nullptr;
    if (hipStreamCreate(&st) != hipSuccess) fail("hipStreamCreate");
    {
      const auto& hy = model.hypers();
      const pet::HostEdges e = pet::build_edges(s, cutoff, hy.cutoff_width, hy.cutoff_function);
      std::vector<int> z(s.numbers), nb(e.neigh);
      std::vector<double> pos(3 * size_t(N)), cell(9);
      for (int n = 0; n < N; ++n)
        for (int c = 0; c < 3; ++c) pos[3 * size_t(n) + c] = s.positions[n][c];
      for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) cell[3 * r + c] = s.cell[r][c];
      pet::EdgeListView v;
      v.n_atoms = N, v.positions = pos.data(), v.atomic_numbers = z.data(), v.offsets = e.off.data();
      v.neighbors = nb.data(), v.shifts = e.shift.data(), v.cell = cell.data();
      pet::Calculator eager(model, cutoff, s2i, st), graph(model, cutoff, s2i, st, true);
      eager.set_neighbors(v), graph.set_neighbors(v);
      bool same = true;
      auto eq = [](const std::vector<double>& a, const std::vector<double>& b) {
        return a.size() == b.size() && std::memcmp(a.data(), b.data(), sizeof(double) * a.size()) == 0;
      };
      for (int k = 0; k < 10; ++k) {
        // small displacements, so the list stays the one set_neighbors holds
        for (size_t i = 0; i < pos.size(); ++i) pos[i] += 1e-3 * double((i * 7 + k * 3) % 5) - 2e-3;
        const bool f = k % 5 != 4, eg = k % 2 == 0;
        std::vector<double> ga, gb;
        const pet::EnergyResult a = eager.compute_step(pos.data(), cell.data(), f, f && eg ? &ga : nullptr);
        const pet::EnergyResult b = graph.compute_step(pos.data(), cell.data(), f, f && eg ? &gb : nullptr);
        same = same && std::memcmp(&a.total, &b.total, sizeof(double)) == 0 && eq(a.per_atom, b.per_atom) &&
               eq(a.forces, b.forces) && std::memcmp(a.virial, b.virial, sizeof a.virial) == 0 && eq(ga, gb);
      }
      if (graph.graph_broken()) fail("graph capture fell back to eager work");
      if (same) std::fclose(std::fopen((dir + "/graph.ok").c_str(), "wb"));
    }
    (void) hipStreamDestroy(st);

    {  // the dense layer: out = in W^T + b + out
      const int M = 300, Nw = 64, K = 96;
      std::vector<float> A(size_t(M) * K), W(size_t(Nw) * K), b(Nw), C0(size_t(M) * Nw);
      unsigned x = 12345u;
      auto rnd = [&x] { return (x = x * 1664525u + 1013904223u, float(int(x >> 9) - (1 << 22)) / float(1 << 22)); };
      for (float& v : A) v = rnd();
      for (float& v : W) v = rnd();
      for (float& v : b) v = rnd();
      for (float& v : C0) v = rnd();
      float *dA, *dW, *db, *dC;
      if (hipMalloc(&dA, A.size() * 4) || hipMalloc(&dW, W.size() * 4) || hipMalloc(&db, b.size() * 4) ||
          hipMalloc(&dC, C0.size() * 4))
        fail("hipMalloc");
      (void) hipMemcpy(dA, A.data(), A.size() * 4, hipMemcpyHostToDevice);
      (void) hipMemcpy(dW, W.data(), W.size() * 4, hipMemcpyHostToDevice);
      (void) hipMemcpy(db, b.data(), b.size() * 4, hipMemcpyHostToDevice);
      double worst = 0, big = 0;
      const pet::SplitWeights ws(dW, Nw, K, K);
      for (const pet::DenseWeight& dw : {pet::plain_weight(dW, Nw, K, K), ws.weight()}) {
        (void) hipMemcpy(dC, C0.data(), C0.size() * 4, hipMemcpyHostToDevice);
        pet::linear_fused(dC, Nw, dA, K, M, dw, db, 1.0f);
        std::vector<float> C(C0.size());
        (void) hipMemcpy(C.data(), dC, C.size() * 4, hipMemcpyDeviceToHost);
        for (int i = 0; i < M; ++i)
          for (int j = 0; j < Nw; ++j) {
            double ref = double(b[j]) + double(C0[size_t(i) * Nw + j]);
            for (int k = 0; k < K; ++k) ref += double(A[size_t(i) * K + k]) * double(W[size_t(j) * K + k]);
            worst = std::max(worst, std::fabs(ref - double(C[size_t(i) * Nw + j])));
            big = std::max(big, std::fabs(ref));
          }
      }
      (void) hipFree(dA), (void) hipFree(dW), (void) hipFree(db), (void) hipFree(dC);
      if (worst <= 1e-5 * big) std::fclose(std::fopen((dir + "/linear.ok").c_str(), "wb"));
    }
    {  // pair rows: dense_pairs gives dense's bits on the split weights (K >= 256)
      const int M = 1000, Nw = 640, K = 256;
      std::vector<float> A(size_t(M) * K), W(size_t(Nw) * K), b(Nw);
      unsigned x = 777u;
      auto rnd = [&x] { return (x = x * 1664525u + 1013904223u, float(int(x >> 9) - (1 << 22)) / float(1 << 22)); };
      for (float& v : A) v = rnd();
      for (float& v : W) v = rnd();
      for (float& v : b) v = rnd();
      float *dA, *dW, *db, *dC;
      if (hipMalloc(&dA, A.size() * 4) || hipMalloc(&dW, W.size() * 4) || hipMalloc(&db, b.size() * 4) ||
          hipMalloc(&dC, size_t(2) * M * Nw * 4))
        fail("hipMalloc");
      (void) hipMemcpy(dA, A.data(), A.size() * 4, hipMemcpyHostToDevice);
      (void) hipMemcpy(dW, W.data(), W.size() * 4, hipMemcpyHostToDevice);
      (void) hipMemcpy(db, b.data(), b.size() * 4, hipMemcpyHostToDevice);
      const pet::SplitWeights ws(dW, Nw, K, K);
      const pet::PairRows ap(dA, M, K, K);
      float* dC2 = dC + size_t(M) * Nw;
      pet::dense(M, dA, K, ws.weight(), dC, Nw, nullptr, db, nullptr, 0, 0.f, nullptr, 0, 1, nullptr);
      pet::dense_pairs(ap, ws.weight(), dC2, Nw, nullptr, db, nullptr, 0, 0.f, nullptr, 0, 1, nullptr);
      std::vector<float> C(size_t(2) * M * Nw);
      (void) hipMemcpy(C.data(), dC, C.size() * 4, hipMemcpyDeviceToHost);
      (void) hipFree(dA), (void) hipFree(dW), (void) hipFree(db), (void) hipFree(dC);
      if (std::memcmp(C.data(), C.data() + size_t(M) * Nw, size_t(M) * Nw * 4) == 0)
        std::fclose(std::fopen((dir + "/pairs.ok").c_str(), "wb"));
    }
  } catch (const std::exception& e) {
    fail(e.what());
  }
  return 0;
}
