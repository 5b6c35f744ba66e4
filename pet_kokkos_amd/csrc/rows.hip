// The attention's input side on gfx950: the cf_seq bias source and the token
// norm (RMSNorm / LayerNorm) forward and backward of the reference's norm_rows /
// norm_rows_bwd (peterspackman/pet-kokkos src/ops.hpp:182-436) and pet_cfseq
// (src/device_neighbors.cpp:318-323).
//
// A norm is HBM-bound (one read and one write of a [rows, width] matrix, a few
// flops an element), so the layout is the one that streams: a wavefront per
// row, lane l holding columns l + 64 j in registers (each load instruction a
// coalesced 256-byte segment), the row's sums a butterfly over the 64 lanes
// that leaves every lane the same bits, four rows a 256-thread workgroup. A
// row is read from memory once.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "../../include/pet_attn.h"

namespace pet_rows {

constexpr float kRmsEps = 1.1920928955078125e-07f;  // float32 epsilon (src/ops.hpp:195)
constexpr float kLnEps = 1e-5f;                      // (src/ops.hpp:196)

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// a * b rounded on its own, never contracted into a following add.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }

// out = norm(in): V columns a lane (V = ceil(width / 64)), masked past width.
template <int V>
__global__ void __launch_bounds__(256) norm_fwd_kernel(int rows, int width, float* __restrict__ out, int64_t ldo,
                                                       const float* __restrict__ in, int64_t ldi,
                                                       const float* __restrict__ weight,
                                                       const float* __restrict__ bias) {
  const int r = blockIdx.x * 4 + int(threadIdx.x >> 6), l = threadIdx.x & 63;
  if (r >= rows) return;
  const bool ln = bias != nullptr;
  const float* x_row = in + int64_t(r) * ldi;
  float x[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    x[j] = d < width ? x_row[d] : 0.0f;
  }
  float mu = 0.0f;
  if (ln) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += x[j];
    mu = wave_sum(s) / width;
  }
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j)
    if (l + 64 * j < width) v += (x[j] - mu) * (x[j] - mu);
  v = wave_sum(v);
  const float inv = 1.0f / sqrtf(v / width + (ln ? kLnEps : kRmsEps));
  float* o_row = out + int64_t(r) * ldo;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    if (d < width) o_row[d] = (x[j] - mu) * inv * weight[d] + (ln ? bias[d] : 0.0f);
  }
}

// in_adj = beta in_adj + the norm's adjoint, with beta_node for rows < n_node
// and beta_edge for the rows after; rows at or past live_end are left alone.
template <int V>
__global__ void __launch_bounds__(256) norm_bwd_kernel(int rows, int width, float* __restrict__ in_adj, int64_t lda,
                                                       const float* __restrict__ out_adj, int64_t ldg,
                                                       const float* __restrict__ in, int64_t ldi,
                                                       const float* __restrict__ weight, int ln, int n_node,
                                                       float beta_node, float beta_edge,
                                                       const int* __restrict__ live_off) {
  const int r = blockIdx.x * 4 + int(threadIdx.x >> 6), l = threadIdx.x & 63;
  if (r >= rows) return;
  if (live_off && r >= n_node + live_off[n_node]) return;  // a capacity's dead row: no sink
  const float beta = r < n_node ? beta_node : beta_edge;
  const float* x_row = in + int64_t(r) * ldi;
  const float* g_row = out_adj + int64_t(r) * ldg;
  float x[V], ga[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    x[j] = d < width ? x_row[d] : 0.0f;
    ga[j] = d < width ? g_row[d] : 0.0f;
  }
  float mu = 0.0f;
  if (ln) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < V; ++j) s += x[j];
    mu = wave_sum(s) / width;
  }
  float sq = 0.0f, sg = 0.0f, sgx = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    if (d < width) {
      const float xv = x[j] - mu, gw = ga[j] * weight[d];
      sq += xv * xv;
      sg += gw;
      sgx += gw * xv;
    }
  }
  sq = wave_sum(sq), sg = wave_sum(sg), sgx = wave_sum(sgx);
  const float inv = 1.0f / sqrtf(sq / width + (ln ? kLnEps : kRmsEps));
  const float mg = ln ? sg / width : 0.0f, mgx = sgx * inv / width;
  float* a_row = in_adj + int64_t(r) * lda;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    if (d < width) {
      // inv (g w - mg - xhat mgx), xhat = (x - mu) inv, as fma(-xhat, mgx, fma(g, w, -mg))
      const float a = fmaf(ga[j], weight[d], -mg), b = mul_rn(x[j] - mu, inv);
      const float g = mul_rn(inv, fmaf(-b, mgx, a));
      a_row[d] = beta == 0.0f ? g : beta * a_row[d] + g;
    }
  }
}

template <class F>
int with_lanes(int width, F&& f) {
  const int v = (width + 63) / 64;
  if (v <= 1) return f(std::integral_constant<int, 1>{});
  if (v <= 2) return f(std::integral_constant<int, 2>{});
  if (v <= 4) return f(std::integral_constant<int, 4>{});
  if (v <= 8) return f(std::integral_constant<int, 8>{});
  if (v <= 16) return f(std::integral_constant<int, 16>{});
  if (v <= 32) return f(std::integral_constant<int, 32>{});
  return PET_ATTN_EINVAL;  // wider than 2048
}

__global__ void cf_seq_kernel(int N, int S, const int* __restrict__ off, const float* __restrict__ cut,
                              float* __restrict__ cf_seq, int64_t ldc) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(N) * S) return;
  const int n = int(i / S), s = int(i - int64_t(n) * S);
  const int e0 = off[n], cnt = off[n + 1] - e0 + 1;
  cf_seq[int64_t(n) * ldc + s] = s == 0 ? 1.0f : s < cnt ? cut[e0 + s - 1] : 0.0f;
}

// inv[r] = 1 / sqrt(mean(in[r]^2) + eps): RMSNorm's row factor, the same
// reductions and arithmetic as norm_fwd_kernel's.
template <int V>
__global__ void __launch_bounds__(256) rms_inv_kernel(int rows, int width, const float* __restrict__ in, int64_t ldi,
                                                      float* __restrict__ inv) {
  const int r = blockIdx.x * 4 + int(threadIdx.x >> 6), l = threadIdx.x & 63;
  if (r >= rows) return;
  const float* x_row = in + int64_t(r) * ldi;
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int d = l + 64 * j;
    const float x = d < width ? x_row[d] : 0.0f;
    if (d < width) v += x * x;
  }
  v = wave_sum(v);
  if (l == 0) inv[r] = 1.0f / sqrtf(v / width + kRmsEps);
}

// out[o][d] = w[o][d] * s[d]: a norm weight folded into the linear after it.
__global__ void fold_cols_kernel(float* __restrict__ out, const float* __restrict__ w, const float* __restrict__ s,
                                 int rows, int cols) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < int64_t(rows) * cols) out[i] = w[i] * s[i % cols];
}

}  // namespace pet_rows

using namespace pet_rows;

// Internal entry of the norm's backward with the reference's sink (node rows
// set with beta_node, edge rows accumulated with beta_edge, dead rows left):
// used by the op level.
int pet_rows_norm_bwd_sink(int rows, int width, float* in_adj, int64_t lda, const float* out_adj, int64_t ldg,
                           const float* in, int64_t ldi, const float* weight, int ln, int n_node, float beta_node,
                           float beta_edge, const int* live_off, hipStream_t st) {
  if (rows < 0 || width < 1) return PET_ATTN_EINVAL;
  if (!in_adj || !out_adj || !in || !weight || lda < width || ldg < width || ldi < width) return PET_ATTN_EINVAL;
  if (rows == 0) return PET_ATTN_OK;
  return with_lanes(width, [&](auto vc) {
    constexpr int V = decltype(vc)::value;
    hipLaunchKernelGGL(norm_bwd_kernel<V>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, rows, width, in_adj, lda,
                       out_adj, ldg, in, ldi, weight, ln, n_node, beta_node, beta_edge, live_off);
    return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
  });
}

int pet_rows_rms_inv(int rows, int width, const float* in, int64_t ldi, float* inv, hipStream_t st) {
  if (rows < 0 || width < 1 || !in || !inv || ldi < width) return PET_ATTN_EINVAL;
  if (rows == 0) return PET_ATTN_OK;
  return with_lanes(width, [&](auto vc) {
    constexpr int V = decltype(vc)::value;
    hipLaunchKernelGGL(rms_inv_kernel<V>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, rows, width, in, ldi, inv);
    return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
  });
}

int pet_rows_fold_cols(float* out, const float* w, const float* s, int rows, int cols, hipStream_t st) {
  const int64_t n = int64_t(rows) * cols;
  if (n == 0) return PET_ATTN_OK;
  hipLaunchKernelGGL(fold_cols_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, out, w, s, rows, cols);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

extern "C" {

int pet_attn_cf_seq(const pet_attn_shape* sh, const int* off, const float* cut, float* cf_seq, int64_t ldc,
                    void* stream) {
  if (!sh || sh->n_atoms < 0 || sh->slots < 1 || !off || !cf_seq || ldc < sh->slots) return PET_ATTN_EINVAL;
  const int64_t total = int64_t(sh->n_atoms) * sh->slots;
  if (total == 0) return PET_ATTN_OK;
  if (!cut && sh->n_rows > sh->n_atoms) return PET_ATTN_EINVAL;
  hipLaunchKernelGGL(cf_seq_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), sh->n_atoms, sh->slots, off, cut, cf_seq, ldc);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

int pet_norm_rows(int rows, int width, float* out, int64_t ldo, const float* in, int64_t ldi, const float* weight,
                  const float* bias, void* stream) {
  if (rows < 0 || width < 1 || !out || !in || !weight || ldo < width || ldi < width) return PET_ATTN_EINVAL;
  if (rows == 0) return PET_ATTN_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return with_lanes(width, [&](auto vc) {
    constexpr int V = decltype(vc)::value;
    hipLaunchKernelGGL(norm_fwd_kernel<V>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, rows, width, out, ldo,
                       in, ldi, weight, bias);
    return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
  });
}

int pet_norm_rows_bwd(int rows, int width, float* in_adj, int64_t lda, float beta, const float* out_adj, int64_t ldg,
                      const float* in, int64_t ldi, const float* weight, int ln, void* stream) {
  return pet_rows_norm_bwd_sink(rows, width, in_adj, lda, out_adj, ldg, in, ldi, weight, ln, rows, beta, beta,
                                nullptr, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
