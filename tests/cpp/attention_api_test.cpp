// Drives pet::attention / pet::attention_bwd (include/pet/attention.hpp) as a
// C++ caller of the reference's interface would, for tests/test_gpu_cpp_api.py:
//
//   attention_api_test DIR N T S H HD TEMPERATURE BETA D_IN
//
// reads DIR/{qkv,cf,w_in,w_out,b_out,out_adj,in_adj0,cf_adj0}.f32 and
// DIR/off.i32 (raw little-endian arrays), runs the forward (save) and the
// backward twice on a warm workspace, and writes DIR/{out,in_adj,cf_adj}.f32
// of the first backward plus DIR/repeat.ok when the second is bit-identical.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "pet/attention.hpp"

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

int main(int argc, char** argv) {
  if (argc != 10) {
    std::fprintf(stderr, "usage: %s DIR N T S H HD TEMPERATURE BETA D_IN\n", argv[0]);
    return 1;
  }
  const std::string dir = argv[1];
  const int N = std::atoi(argv[2]), T = std::atoi(argv[3]), S = std::atoi(argv[4]), H = std::atoi(argv[5]),
            HD = std::atoi(argv[6]), d_in = std::atoi(argv[9]);
  const double temperature = std::atof(argv[7]);
  const float beta = float(std::atof(argv[8]));
  const int D = H * HD;
  auto qkv = read<float>(dir + "/qkv.f32", size_t(T) * 3 * D);
  auto cf = read<float>(dir + "/cf.f32", size_t(N) * S);
  auto off = read<int>(dir + "/off.i32", size_t(N) + 1);
  auto w_in = read<float>(dir + "/w_in.f32", size_t(3) * D * d_in);
  auto w_out = read<float>(dir + "/w_out.f32", size_t(D) * D);
  auto b_out = read<float>(dir + "/b_out.f32", size_t(D));
  auto out_adj = read<float>(dir + "/out_adj.f32", size_t(T) * D);
  auto in_adj0 = read<float>(dir + "/in_adj0.f32", size_t(T) * d_in);
  auto cf_adj0 = read<float>(dir + "/cf_adj0.f32", size_t(N) * S);

  float *d_qkv = dev(qkv), *d_cf = dev(cf), *d_w_in = dev(w_in), *d_w_out = dev(w_out), *d_b_out = dev(b_out);
  float *d_out_adj = dev(out_adj), *d_out = dev(std::vector<float>(size_t(T) * D));
  int* d_off = dev(off);
  pet::Workspace ws;
  pet::Tokens tk;
  tk.off = d_off, tk.N = N;
  std::vector<std::vector<float>> results;
  try {
    pet::attention(ws, "L0.a0", pet::View2D(d_out, T, D), pet::View2D(d_qkv, T, 3 * D), pet::View2D(d_cf, N, S),
                   pet::WeightRef(pet::View2D(d_w_out, D, D)), pet::View1D{d_b_out, D}, tk, S, H, HD, temperature,
                   true);
    for (int rep = 0; rep < 2; ++rep) {
      float* d_in_adj = dev(in_adj0);
      float* d_cf_adj = dev(cf_adj0);
      pet::attention_bwd(ws, "L0.a0", pet::View2D(d_in_adj, T, d_in), pet::View2D(d_cf_adj, N, S),
                         pet::View2D(d_out_adj, T, D), pet::View2D(d_qkv, T, 3 * D), pet::View2D(d_cf, N, S),
                         pet::WeightRef(pet::View2D(d_w_in, 3 * D, d_in)), pet::WeightRef(pet::View2D(d_w_out, D, D)),
                         tk, S, H, HD, temperature, beta);
      if (hipDeviceSynchronize() != hipSuccess) return 6;
      results.push_back(host(d_in_adj, size_t(T) * d_in));
      results.push_back(host(d_cf_adj, size_t(N) * S));
      (void) hipFree(d_in_adj);
      (void) hipFree(d_cf_adj);
    }
    // a backward with no saved forward must throw
    bool threw = false;
    try {
      pet::attention_bwd(ws, "missing", pet::View2D(d_out, T, D), pet::View2D(d_cf, N, S),
                         pet::View2D(d_out_adj, T, D), pet::View2D(d_qkv, T, 3 * D), pet::View2D(d_cf, N, S),
                         pet::WeightRef(pet::View2D(d_w_in, 3 * D, d_in)), pet::WeightRef(pet::View2D(d_w_out, D, D)),
                         tk, S, H, HD, temperature, beta);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    if (!threw) return 7;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 8;
  }
  write(dir + "/out.f32", host(d_out, size_t(T) * D));
  write(dir + "/in_adj.f32", results[0]);
  write(dir + "/cf_adj.f32", results[1]);
  if (std::memcmp(results[0].data(), results[2].data(), results[0].size() * 4) == 0 &&
      std::memcmp(results[1].data(), results[3].data(), results[1].size() * 4) == 0)
    write(dir + "/repeat.ok", std::vector<char>{'1'});
  std::printf("ok\n");
  return 0;
}
