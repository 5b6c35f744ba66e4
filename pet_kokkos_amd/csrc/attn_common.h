// Device pieces shared by the attention kernels (attention.hip, the
// LDS-staged kernels; attention_stream.hip, the streaming ones): the MFMA and
// lane-exchange primitives, the mask constants, qkv loads with the fused
// transform, and an (atom, head) work item's token rows.
//
// Reference semantics: peterspackman/pet-kokkos src/attention.cpp:1-16,
// :54-55 (kOff and the off test), src/ops.hpp:31-37 (the token rows).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pet_attn {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr float kOff = -1e30f;  // the log cf of a key no query sees
// log cf of a key with cf > 0: the hardware log2 times ln 2 (the fast log of
// the reference's device path), held above -104 (log of the smallest
// subnormal) so that a subnormal cf, which the hardware log flushes, stays a
// live key.
__device__ __forceinline__ float log_cf(float cf) {
  return fmaxf(__builtin_amdgcn_logf(cf) * 0.693147180559945309f, -104.f);
}
__device__ __forceinline__ bool is_off(float lc) { return lc < -1e29f; }
// The running max's start in the matrix-core forward: above kOff, so a key
// with log cf kOff has exp(x - max) = 0 exactly whatever keys came before,
// without a test per key (x = s sc + kOff rounds to kOff for any real score).
constexpr float kFloor = -1e29f;

// Over the four lanes that share c (g = 0..3): gfx950's lane-swap
// instructions exchange rows of 32 and of 16 lanes in registers, no LDS. Both
// lanes of a pair combine the same two values in the same order, so every
// lane ends with bit-identical results.
__device__ __forceinline__ float max_g(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_g(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// A workgroup barrier that orders LDS traffic only. __syncthreads() also
// fences global memory, which on gfx9 means waiting for every outstanding
// vector-memory load -- the prefetches a barrier is meant to overlap.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// n floats from LDS (p aligned to n floats when n is 2 or 4).
template <int n>
__device__ __forceinline__ void lds_get(const float* p, float* out) {
  if constexpr (n % 4 == 0) {
#pragma unroll
    for (int j = 0; j < n; j += 4) {
      const float4 x = *reinterpret_cast<const float4*>(p + j);
      out[j] = x.x, out[j + 1] = x.y, out[j + 2] = x.z, out[j + 3] = x.w;
    }
  } else if constexpr (n % 2 == 0) {
#pragma unroll
    for (int j = 0; j < n; j += 2) {
      const float2 x = *reinterpret_cast<const float2*>(p + j);
      out[j] = x.x, out[j + 1] = x.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < n; ++j) out[j] = p[j];
  }
}
// n (a multiple of 4) floats from global memory, 16-byte aligned.
template <int n>
__device__ __forceinline__ void gmem_get(const float* p, float* out) {
#pragma unroll
  for (int j = 0; j < n; j += 4) {
    const float4 x = *reinterpret_cast<const float4*>(p + j);
    out[j] = x.x, out[j + 1] = x.y, out[j + 2] = x.z, out[j + 3] = x.w;
  }
}

// An affine map of qkv applied as it is loaded: row r's values scaled by
// rs[r], then column j's bias b[j] added (either may be null). With qkv the
// product of raw tokens and the input linear whose weight has the RMSNorm
// weight folded in, rs = 1/rms(token) and b the linear's bias make it
// norm(tokens) W^T + b without the normed tokens or the bias pass ever
// touching memory: the QKV projection's epilogue, fused into its consumer.
struct QkvXf {
  const float* rs = nullptr;
  const float* b = nullptr;
};
template <int W, bool XF>
__device__ __forceinline__ void qkv_get(const float* qkv, int64_t ldq, size_t r, int col, const QkvXf& xf,
                                        float* out) {
  gmem_get<W>(qkv + r * ldq + col, out);
  if constexpr (!XF) return;
  if (xf.rs) {
    const float sc = xf.rs[r];
#pragma unroll
    for (int t = 0; t < W; ++t) out[t] *= sc;
  }
  if (xf.b) {
    float bb[W];
    gmem_get<W>(xf.b + col, bb);
#pragma unroll
    for (int t = 0; t < W; ++t) out[t] += bb[t];
  }
}

// The work item of workgroup b of a one-item-per-workgroup grid of `items`,
// XCD-grouped: the dispatcher hands workgroup b to XCD b % 8, so XCD x gets
// workgroups x, x + 8, ... and, with this map, the contiguous items
// [x q + min(x, r), ...) (q = items / 8, r = items % 8): the heads of an atom
// and its neighbour atoms' rows run on one XCD close in time, so the 128-byte
// head slices of a token's rows meet in one L2 and reach HBM as whole rows.
// Measured on the backward's access pattern alone at C3: 232 -> 205 us.
__device__ __forceinline__ int xcd_item(int b, int items) {
  const int x = b & 7, k = b >> 3, q = items >> 3, r = items & 7;
  return x * q + (x < r ? x : r) + k;
}

// One work item, an (atom, head), of a run of atoms [n0, n1). The atom's
// tokens are rows of two matrices: the whole token matrix (merged, and the
// per-slot arrays), and the run's chunk (qkv, dO, qkv_adj), which holds the
// run's own rows first (atom n at n - n0) and then its edges' rows (edge k at
// eb + k, eb = (n1 - n0) - off[n0]). Unchunked, n0 = 0 and eb = N and the two
// agree (the chunk layout of the reference's attention_chunked,
// src/attention.cpp:2055-2070, run_qkv).
struct Atom {
  int n, h, N, n0, o0, cnt, nb;
  int64_t eb;
  __device__ Atom(const int* off, int item, int H, int N_, int S, int n0_, int64_t eb_) : N(N_), n0(n0_), eb(eb_) {
    const int a = item / H;
    h = item - a * H;
    n = n0 + a;
    o0 = off[n];
    const int c = off[n + 1] - o0 + 1;
    cnt = c < S ? c : S;  // a count above S would be the caller's error; never read past S
    nb = (cnt + 15) >> 4;
  }
  // slot s's row in the run's chunk
  __device__ size_t row(int s) const { return s == 0 ? size_t(n - n0) : size_t(eb + o0 + s - 1); }
  // slot s's row in the whole token matrix
  __device__ size_t grow(int s) const { return s == 0 ? size_t(n) : size_t(N) + size_t(o0) + size_t(s - 1); }
};

// Element e of a lane's hd/4 slice, from the DT result tiles: e = r * DT + t.
template <int DT>
__device__ __forceinline__ float tile_elem(const f4* acc, int e) {
  return acc[e % DT][e / DT];
}
template <int HD>
__device__ __forceinline__ void store_slice(float* dst, const f4* acc, float f) {
  constexpr int W = HD / 4, DT = HD / 16;
#pragma unroll
  for (int e = 0; e < W; e += 4)
    *reinterpret_cast<float4*>(dst + e) =
        make_float4(tile_elem<DT>(acc, e) * f, tile_elem<DT>(acc, e + 1) * f, tile_elem<DT>(acc, e + 2) * f,
                    tile_elem<DT>(acc, e + 3) * f);
}


}  // namespace pet_attn
