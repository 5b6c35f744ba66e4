// pet/attention.hpp -- the reference's C++ attention interface over the C ABI.
//
// pet::attention and pet::attention_bwd (and the token norm, cf_seq and the
// layer-level attention block around them) with the arguments, meaning, conventions
// and error behaviour of peterspackman/pet-kokkos's (src/ops.hpp:121-132,
// src/attention.cpp:2189-2206), for a caller that holds plain device pointers
// instead of Kokkos views:
//   - View2D is a row-major device matrix with its own row stride
//     (Kokkos::View<float**, LayoutRight> sliced as the reference does);
//   - WeightRef is a torch-Linear-layout weight [out, in];
//   - Tokens is the CSR layout of src/ops.hpp:31-37 (off on the device);
//   - Workspace keeps named device buffers between calls, as the reference's
//     (include/pet/kokkos.hpp:65-235): the forward saves merged and ml under
//     key + ":merged" / key + ":ml", the backward finds them by the same key
//     (peek2) and takes its scratch from the pool; a warm call allocates
//     nothing;
//   - errors throw std::runtime_error with the C ABI's message.
// Every kernel runs in libpet_attn.so (HIP, gfx950) on `stream`.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>

#include "../pet_attn.h"

namespace pet {

using Net = float;

struct View2D {
  float* ptr = nullptr;
  int rows = 0, cols = 0;
  int64_t ld = 0;  // row stride in elements
  View2D() = default;
  View2D(float* p, int r, int c, int64_t stride = -1) : ptr(p), rows(r), cols(c), ld(stride < 0 ? c : stride) {}
  float* data() const { return ptr; }
  int extent(int d) const { return d == 0 ? rows : cols; }
  int64_t stride(int d) const { return d == 0 ? ld : 1; }
};
struct View1D {
  float* ptr = nullptr;
  int n = 0;
  float* data() const { return ptr; }
};
struct WeightRef {
  View2D v;  // [out, in], contiguous
  WeightRef() = default;
  explicit WeightRef(const View2D& m) : v(m) {}
  int extent(int d) const { return v.extent(d); }
};
struct Tokens {
  const int* off = nullptr;  // device, N + 1 entries
  int N = 0;
  bool dead = false;  // edge rows past N + off[N] may exist (a capacity)
};

inline void check(int code, const char* what) {
  if (code != PET_ATTN_OK) throw std::runtime_error(std::string("pet: ") + what + ": " + pet_attn_strerror(code));
}

class Workspace {
 public:
  Workspace() = default;
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;
  ~Workspace() { release(); }

  // A named [r, c] buffer, grown when too small and otherwise reused.
  View2D n2(const std::string& k, int r, int c) {
    float* p = static_cast<float*>(bytes(k, sizeof(float) * size_t(r) * size_t(c)));
    return cur2_[k] = View2D(p, r, c);
  }
  // The view the last n2(k, ...) handed out: a saved activation.
  View2D peek2(const std::string& k) const {
    auto it = cur2_.find(k);
    if (it == cur2_.end()) throw std::runtime_error("pet: workspace has no buffer named '" + k + "'");
    return it->second;
  }
  // A named buffer of at least n bytes (256-byte aligned, as hipMalloc's).
  void* bytes(const std::string& k, size_t n) {
    Buf& b = named_[k];
    if (b.size < n) {
      if (b.ptr) check(hipFree(b.ptr) == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH, "hipFree");
      b.ptr = nullptr;
      const size_t grow = b.size ? n + n / 4 : n;
      if (hipMalloc(&b.ptr, grow) != hipSuccess) throw std::runtime_error("pet: workspace allocation failed");
      b.size = grow;
    }
    return b.ptr;
  }
  void release() {
    for (auto& kv : named_)
      if (kv.second.ptr) (void) hipFree(kv.second.ptr);
    named_.clear();
    cur2_.clear();
  }

 private:
  struct Buf {
    void* ptr = nullptr;
    size_t size = 0;
  };
  std::map<std::string, Buf> named_;
  std::map<std::string, View2D> cur2_;
};

inline pet_attn_shape make_shape(const Tokens& tk, int T, int S, int heads, int head_dim, double temperature) {
  pet_attn_shape sh;
  sh.n_atoms = tk.N;
  sh.n_rows = T;
  sh.slots = S;
  sh.heads = heads;
  sh.head_dim = head_dim;
  sh.dead = tk.dead ? 1 : 0;
  sh.scale = pet_attn_scale(head_dim, temperature);
  return sh;
}

// Multi-head attention over each atom's tokens with log(cf) as a per-key bias,
// then out = merged W_out^T + b_out. `save` keeps what the backward needs under
// `key`.
inline void attention(Workspace& ws, const std::string& key, View2D out, View2D qkv, View2D cf_seq,
                      const WeightRef& w_out, View1D b_out, const Tokens& tk, int S, int heads, int head_dim,
                      double temperature, bool save, hipStream_t stream = nullptr) {
  const int D = heads * head_dim, T = qkv.extent(0);
  if (cf_seq.extent(1) < S) throw std::runtime_error("pet: cf_seq narrower than S");
  const View2D merged = ws.n2(save ? key + ":merged" : std::string("attention:tmp"), T, D);
  float* ml = save ? ws.n2(key + ":ml", tk.N * heads * S, 2).data() : nullptr;
  const pet_attn_shape sh = make_shape(tk, T, S, heads, head_dim, temperature);
  check(pet_attention(&sh, out.data(), out.stride(0), qkv.data(), qkv.stride(0), cf_seq.data(), cf_seq.stride(0),
                      w_out.v.data(), b_out.data(), tk.off, merged.data(), ml, stream),
        "attention");
}

// in_adj (onto beta * in_adj) is the adjoint of the input linear's input;
// cf_seq_adj accumulates. `key` names the forward's saves.
inline void attention_bwd(Workspace& ws, const std::string& key, View2D in_adj, View2D cf_seq_adj, View2D out_adj,
                          View2D qkv, View2D cf_seq, const WeightRef& w_in, const WeightRef& w_out, const Tokens& tk,
                          int S, int heads, int head_dim, double temperature, Net beta,
                          hipStream_t stream = nullptr) {
  const int T = qkv.extent(0);
  const View2D merged = ws.peek2(key + ":merged"), ml = ws.peek2(key + ":ml");
  const pet_attn_shape sh = make_shape(tk, T, S, heads, head_dim, temperature);
  const size_t need = pet_attention_bwd_workspace(&sh);
  void* scratch = ws.bytes("attention_bwd:scratch", need);
  check(pet_attention_bwd(&sh, in_adj.data(), in_adj.stride(0), w_in.extent(1), cf_seq_adj.data(),
                          cf_seq_adj.stride(0), out_adj.data(), out_adj.stride(0), qkv.data(), qkv.stride(0),
                          cf_seq.data(), cf_seq.stride(0), w_in.v.data(), w_out.v.data(), tk.off, merged.data(),
                          ml.data(), beta, scratch, need, stream),
        "attention_bwd");
}

// ---- the attention's input side ------------------------------------------

// cf_seq [N, S]: 1, then the atom's kept edges' cutoff factors (cut, packed
// order), then 0 (the reference's pet_cfseq, src/device_neighbors.cpp:318-323).
inline void cf_seq(View2D out, const Tokens& tk, const float* cut, int S, hipStream_t stream = nullptr) {
  pet_attn_shape sh = make_shape(tk, tk.N, S, 1, 16, 1.0);
  sh.n_rows = tk.N + (cut ? 1 : 0);
  check(pet_attn_cf_seq(&sh, tk.off, cut, out.data(), out.stride(0), stream), "cf_seq");
}

// out = norm(in) row by row: RMSNorm, or LayerNorm when bias has data
// (norm_rows, src/ops.hpp:376-407, with the identity prologue).
inline void norm_rows(View2D out, View2D in, View1D weight, View1D bias, hipStream_t stream = nullptr) {
  check(pet_norm_rows(in.extent(0), in.extent(1), out.data(), out.stride(0), in.data(), in.stride(0), weight.data(),
                      bias.data(), stream),
        "norm_rows");
}

// in_adj = beta in_adj + the norm's input adjoint (norm_rows_bwd,
// src/ops.hpp:409-436, with the sink "in_adj(r, d) = beta in_adj + g").
inline void norm_rows_bwd(View2D in_adj, View2D out_adj, View2D in, View1D weight, bool ln, Net beta = 0,
                          hipStream_t stream = nullptr) {
  check(pet_norm_rows_bwd(in.extent(0), in.extent(1), in_adj.data(), in_adj.stride(0), beta, out_adj.data(),
                          out_adj.stride(0), in.data(), in.stride(0), weight.data(), ln ? 1 : 0, stream),
        "norm_rows_bwd");
}

// The attention block of a PET layer from its tokens (PetModel::ff_layer,
// src/feedforward.cpp:96-123): norm, qkv = linear(normed, w_in, b_in),
// attention; the saves under `key`.
inline void attention_layer(Workspace& ws, const std::string& key, View2D out, View2D tokens, View1D norm_w,
                            View1D norm_b, const WeightRef& w_in, View1D b_in, View2D cf_seq, const WeightRef& w_out,
                            View1D b_out, const Tokens& tk, int S, int heads, int head_dim, double temperature,
                            hipStream_t stream = nullptr) {
  const int D = heads * head_dim, T = tokens.extent(0);
  const pet_attn_shape sh = make_shape(tk, T, S, heads, head_dim, temperature);
  const View2D merged = ws.n2(key + ":merged", T, D);
  const View2D ml = ws.n2(key + ":ml", tk.N * heads * S, 2);
  const size_t need = pet_attention_layer_workspace(&sh);
  void* scratch = ws.bytes("attention_layer:scratch", need);
  check(pet_attention_layer(&sh, out.data(), out.stride(0), tokens.data(), tokens.stride(0), norm_w.data(),
                            norm_b.data(), w_in.v.data(), b_in.data(), cf_seq.data(), cf_seq.stride(0),
                            w_out.v.data(), b_out.data(), tk.off, merged.data(), ml.data(), scratch, need, stream),
        "attention_layer");
}

// Its backward (PetModel::ff_layer_bwd, src/feedforward.cpp:292-329): the
// tokens' adjoint, atom rows set and live edge rows accumulated as the
// reference's sink does; cf_seq_adj accumulates.
inline void attention_layer_bwd(Workspace& ws, const std::string& key, View2D tokens_adj, View2D cf_seq_adj,
                                View2D out_adj, View2D tokens, View1D norm_w, View1D norm_b, const WeightRef& w_in,
                                View1D b_in, View2D cf_seq, const WeightRef& w_out, const Tokens& tk, int S,
                                int heads, int head_dim, double temperature, hipStream_t stream = nullptr) {
  const int T = tokens.extent(0);
  const pet_attn_shape sh = make_shape(tk, T, S, heads, head_dim, temperature);
  const View2D merged = ws.peek2(key + ":merged"), ml = ws.peek2(key + ":ml");
  const size_t need = pet_attention_layer_workspace(&sh);
  void* scratch = ws.bytes("attention_layer:scratch", need);
  check(pet_attention_layer_bwd(&sh, tokens_adj.data(), tokens_adj.stride(0), cf_seq_adj.data(), cf_seq_adj.stride(0),
                                out_adj.data(), out_adj.stride(0), tokens.data(), tokens.stride(0), norm_w.data(),
                                norm_b.data(), w_in.v.data(), b_in.data(), cf_seq.data(), cf_seq.stride(0),
                                w_out.v.data(), tk.off, merged.data(), ml.data(), scratch, need, stream),
        "attention_layer_bwd");
}

}  // namespace pet
