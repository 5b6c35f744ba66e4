// Drives the layer-level attention and the forces' edge term through the C++
// interface (include/pet/attention.hpp, include/pet/forces.hpp) as a C++
// caller of the reference's would, for tests/test_gpu_cpp_api.py:
//
//   layer_forces_test DIR N T S H HD E
//
// reads DIR/{tokens,nw,w_in,b_in,w_out,b_out,cut,out_adj,x4}.f32,
// DIR/{off,center,reverse}.i32 and DIR/{vec,dist,pcut}.f64, then: cf_seq from
// the edges' cutoff factors, attention_layer, attention_layer_bwd (cf_seq_adj
// from zero) and forces_and_virial (cosine cutoff, width 0.5, scale -1); writes
// DIR/{cf,out,tokens_adj,cf_adj}.f32 and DIR/{forces,vir9,grad}.f64; then runs
// the same chain four more times through a pet::StepRecorder on a stream of its
// own (eager, captured, replayed, replayed) and writes DIR/graph.ok when every
// run gave the first one's bits.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include <cstring>

#include "pet/forces.hpp"
#include "pet/replay.hpp"

template <class T>
static std::vector<T> read(const std::string& path, size_t n) {
  std::vector<T> v(n);
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f || std::fread(v.data(), sizeof(T), n, f) != n) {
    std::fprintf(stderr, "cannot read %s\n", path.c_str());
    std::exit(2);
  }
  std::fclose(f);
  return v;
}
template <class T>
static void write(const std::string& path, const std::vector<T>& v) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) std::exit(3);
  std::fclose(f);
}
template <class T>
static T* dev(const std::vector<T>& h) {
  T* p = nullptr;
  if (hipMalloc(&p, sizeof(T) * (h.size() ? h.size() : 1)) != hipSuccess) std::exit(4);
  if (!h.empty() && hipMemcpy(p, h.data(), sizeof(T) * h.size(), hipMemcpyHostToDevice) != hipSuccess) std::exit(4);
  return p;
}
template <class T>
static std::vector<T> host(const T* p, size_t n) {
  std::vector<T> h(n);
  if (hipMemcpy(h.data(), p, sizeof(T) * n, hipMemcpyDeviceToHost) != hipSuccess) std::exit(5);
  return h;
}

__global__ void fill0(float* p, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = 0.0f;
}

int main(int argc, char** argv) {
  if (argc != 8) {
    std::fprintf(stderr, "usage: %s DIR N T S H HD E\n", argv[0]);
    return 1;
  }
  const std::string dir = argv[1];
  const int N = std::atoi(argv[2]), T = std::atoi(argv[3]), S = std::atoi(argv[4]), H = std::atoi(argv[5]),
            HD = std::atoi(argv[6]), E = std::atoi(argv[7]);
  const int D = H * HD;
  float* tokens = dev(read<float>(dir + "/tokens.f32", size_t(T) * D));
  float* nw = dev(read<float>(dir + "/nw.f32", size_t(D)));
  float* w_in = dev(read<float>(dir + "/w_in.f32", size_t(3) * D * D));
  float* b_in = dev(read<float>(dir + "/b_in.f32", size_t(3) * D));
  float* w_out = dev(read<float>(dir + "/w_out.f32", size_t(D) * D));
  float* b_out = dev(read<float>(dir + "/b_out.f32", size_t(D)));
  float* cut = dev(read<float>(dir + "/cut.f32", size_t(E)));
  float* out_adj = dev(read<float>(dir + "/out_adj.f32", size_t(T) * D));
  float* x4 = dev(read<float>(dir + "/x4.f32", size_t(E) * 4));
  int* off = dev(read<int>(dir + "/off.i32", size_t(N) + 1));
  int* center = dev(read<int>(dir + "/center.i32", size_t(E)));
  int* reverse = dev(read<int>(dir + "/reverse.i32", size_t(E)));
  double* vec = dev(read<double>(dir + "/vec.f64", size_t(E) * 3));
  double* dist = dev(read<double>(dir + "/dist.f64", size_t(E)));
  double* pcut = dev(read<double>(dir + "/pcut.f64", size_t(E)));
  int* soff = dev(std::vector<int>{0, N});
  float* cf = dev(std::vector<float>(size_t(N) * S));
  float* out = dev(std::vector<float>(size_t(T) * D));
  float* tadj = dev(std::vector<float>(size_t(T) * D));
  float* csa = dev(std::vector<float>(size_t(N) * S));
  pet::Workspace ws;
  pet::Tokens tk;
  tk.off = off, tk.N = N;
  pet::PackedEdges pk;
  pk.E = E, pk.n_centres = N, pk.off = off, pk.center = center, pk.reverse = reverse, pk.vec = vec, pk.dist = dist,
  pk.pcut = pcut;
  pet::RView2D forces, vir9, grad;
  try {
    pet::cf_seq(pet::View2D(cf, N, S), tk, cut, S);
    pet::attention_layer(ws, "L0.a0", pet::View2D(out, T, D), pet::View2D(tokens, T, D), pet::View1D{nw, D},
                         pet::View1D{}, pet::WeightRef(pet::View2D(w_in, 3 * D, D)), pet::View1D{b_in, 3 * D},
                         pet::View2D(cf, N, S), pet::WeightRef(pet::View2D(w_out, D, D)), pet::View1D{b_out, D}, tk, S,
                         H, HD, 1.0);
    pet::attention_layer_bwd(ws, "L0.a0", pet::View2D(tadj, T, D), pet::View2D(csa, N, S), pet::View2D(out_adj, T, D),
                             pet::View2D(tokens, T, D), pet::View1D{nw, D}, pet::View1D{},
                             pet::WeightRef(pet::View2D(w_in, 3 * D, D)), pet::View1D{b_in, 3 * D},
                             pet::View2D(cf, N, S), pet::WeightRef(pet::View2D(w_out, D, D)), tk, S, H, HD, 1.0);
    pet::forces_and_virial(ws, pk, N, soff, 1, pet::View2D(x4, E, 4), pet::View1D{}, pet::View2D(csa, N, S), 0.5,
                           pet::CutoffFunction::Cosine, -1.0, forces, vir9, grad);
    if (hipDeviceSynchronize() != hipSuccess) return 6;
    // a bad argument must throw
    bool threw = false;
    try {
      pet::edge_grad(pk, pet::View2D(x4, E, 4), pet::View1D{}, pet::View2D(csa, N, S), 0.5,
                     static_cast<pet::CutoffFunction>(7), grad);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    if (!threw) return 7;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 8;
  }
  write(dir + "/cf.f32", host(cf, size_t(N) * S));
  write(dir + "/out.f32", host(out, size_t(T) * D));
  write(dir + "/tokens_adj.f32", host(tadj, size_t(T) * D));
  write(dir + "/cf_adj.f32", host(csa, size_t(N) * S));
  write(dir + "/forces.f64", host(forces.data(), size_t(N) * 3));
  write(dir + "/vir9.f64", host(vir9.data(), size_t(9)));
  write(dir + "/grad.f64", host(grad.data(), size_t(E) * 3));
  // the chain recorded as a graph and replayed: every run's bits as the first's
  {
    hipStream_t st = nullptr;
    if (hipStreamCreate(&st) != hipSuccess) return 9;
    const auto ref_t = host(tadj, size_t(T) * D);
    const auto ref_c = host(csa, size_t(N) * S);
    const auto ref_f = host(forces.data(), size_t(N) * 3);
    pet::StepRecorder cache(st);
    const pet::Signature key{uint64_t(uintptr_t(tokens)), uint64_t(T), uint64_t(D)};
    bool same = true;
    try {
      for (int rep = 0; rep < 4; ++rep) {
        cache.launch(key, [&] {
          // the accumulated outputs start from zero: a fill kernel, no memset node
          hipLaunchKernelGGL(fill0, dim3(256), dim3(256), 0, st, tadj, size_t(T) * D);
          hipLaunchKernelGGL(fill0, dim3(64), dim3(256), 0, st, csa, size_t(N) * S);
          pet::attention_layer(ws, "L0.a0", pet::View2D(out, T, D), pet::View2D(tokens, T, D), pet::View1D{nw, D},
                               pet::View1D{}, pet::WeightRef(pet::View2D(w_in, 3 * D, D)), pet::View1D{b_in, 3 * D},
                               pet::View2D(cf, N, S), pet::WeightRef(pet::View2D(w_out, D, D)), pet::View1D{b_out, D},
                               tk, S, H, HD, 1.0, st);
          pet::attention_layer_bwd(ws, "L0.a0", pet::View2D(tadj, T, D), pet::View2D(csa, N, S),
                                   pet::View2D(out_adj, T, D), pet::View2D(tokens, T, D), pet::View1D{nw, D},
                                   pet::View1D{}, pet::WeightRef(pet::View2D(w_in, 3 * D, D)),
                                   pet::View1D{b_in, 3 * D}, pet::View2D(cf, N, S),
                                   pet::WeightRef(pet::View2D(w_out, D, D)), tk, S, H, HD, 1.0, st);
          pet::forces_and_virial(ws, pk, N, soff, 1, pet::View2D(x4, E, 4), pet::View1D{}, pet::View2D(csa, N, S),
                                 0.5, pet::CutoffFunction::Cosine, -1.0, forces, vir9, grad, st);
        });
        if (hipStreamSynchronize(st) != hipSuccess) return 10;
        const auto t2 = host(tadj, size_t(T) * D), c2 = host(csa, size_t(N) * S);
        const auto f2 = host(forces.data(), size_t(N) * 3);
        same = same && std::memcmp(t2.data(), ref_t.data(), t2.size() * 4) == 0 &&
               std::memcmp(c2.data(), ref_c.data(), c2.size() * 4) == 0 &&
               std::memcmp(f2.data(), ref_f.data(), f2.size() * 8) == 0;
      }
    } catch (const std::exception& e) {
      std::fprintf(stderr, "graph: %s\n", e.what());
      return 11;
    }
    const auto& n = cache.counters();
    if (same && n.refusals == 0 && n.records == 1 && n.launches == 3 && n.eager == 1 && cache.live() == 1)
      write(dir + "/graph.ok", std::vector<char>{'1'});
    (void) hipStreamDestroy(st);
  }
  std::printf("ok\n");
  return 0;
}
