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

#include "../../include/pet_model.h"
#include "split_bf16.h"

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

// ---- the vectorised row passes ----------------------------------------------
//
// For a width that is a multiple of 4 (rows 16-byte aligned): LPR lanes a row
// (16, 32 or 64: 64 / LPR rows a wavefront), lane t of a row holding float4
// chunks t + LPR j, j < C4, so every load is a 16-byte one and a narrow row
// (128 floats: two a wavefront) does not leave half a wavefront idle. The
// row's sums are a butterfly over its LPR lanes; the arithmetic per value is
// that of the scalar kernels above.
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// PAIRS: the row as fp16 pairs (pair rows: each row scaled by the power of two
// that puts its largest |value| at [2^14, 2^15), 8-value groups of hi then lo
// 16 bytes, the rows' inverse scales after all rows' pairs) into `out`
// instead of fp32: the same values, split as the pair-rows pass would split
// them.
template <int LPR, int C4, bool PAIRS = false>
__global__ void __launch_bounds__(256) norm_fwd4_kernel(int rows, int width, float* __restrict__ out, int64_t ldo,
                                                        const float* __restrict__ in, int64_t ldi,
                                                        const float* __restrict__ weight,
                                                        const float* __restrict__ bias) {
  constexpr int RPW = 64 / LPR;
  const int l = threadIdx.x & 63, t = l % LPR;
  const int r = (blockIdx.x * 4 + int(threadIdx.x >> 6)) * RPW + l / LPR;
  if (r >= rows) return;  // whole row groups exit together: the butterflies stay within live lanes
  const bool ln = bias != nullptr;
  const int w4 = width >> 2;
  const float4* x_row = reinterpret_cast<const float4*>(in + int64_t(r) * ldi);
  float4 x[C4];
#pragma unroll
  for (int j = 0; j < C4; ++j) {
    const int q = t + LPR * j;
    x[j] = q < w4 ? x_row[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mu = 0.0f;
  if (ln) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < C4; ++j) s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
    mu = row_sum<LPR>(s) / width;
  }
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < C4; ++j)
    if (t + LPR * j < w4) {
      const float a = x[j].x - mu, b = x[j].y - mu, c = x[j].z - mu, d = x[j].w - mu;
      v += (a * a + b * b) + (c * c + d * d);
    }
  v = row_sum<LPR>(v);
  const float inv = 1.0f / sqrtf(v / width + (ln ? kLnEps : kRmsEps));
  float4* o_row = reinterpret_cast<float4*>(out + int64_t(r) * ldo);
  const float4* w4p = reinterpret_cast<const float4*>(weight);
  const float4* b4p = reinterpret_cast<const float4*>(bias);
  float4 o[C4];
#pragma unroll
  for (int j = 0; j < C4; ++j) {
    const int q = t + LPR * j;
    if (q < w4) {
      const float4 wq = w4p[q], bq = ln ? b4p[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      o[j] = make_float4((x[j].x - mu) * inv * wq.x + bq.x, (x[j].y - mu) * inv * wq.y + bq.y,
                         (x[j].z - mu) * inv * wq.z + bq.z, (x[j].w - mu) * inv * wq.w + bq.w);
      if constexpr (!PAIRS) o_row[q] = o[j];
    } else {
      o[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if constexpr (PAIRS) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < C4; ++j) m = fmaxf(m, fmaxf(fmaxf(fabsf(o[j].x), fabsf(o[j].y)), fmaxf(fabsf(o[j].z), fabsf(o[j].w))));
#pragma unroll
    for (int k = LPR / 2; k > 0; k >>= 1) m = fmaxf(m, __shfl_xor(m, k));
    const float s = pet_split::pair_scale(m);
    const int KG = width / 8;
    unsigned* base = reinterpret_cast<unsigned*>(out) + int64_t(r) * KG * 8;
#pragma unroll
    for (int j = 0; j < C4; ++j) {
      const int q = t + LPR * j;
      if (q < w4) {
        unsigned h0, h1, l0, l1;
        pet_split::pair2(o[j].x * s, o[j].y * s, h0, l0);
        pet_split::pair2(o[j].z * s, o[j].w * s, h1, l1);
        unsigned* hi = base + (q >> 1) * 8 + (q & 1) * 2;  // group q / 2: hi words 0-3, lo words 4-7
        *reinterpret_cast<uint2*>(hi) = make_uint2(h0, h1);
        *reinterpret_cast<uint2*>(hi + 4) = make_uint2(l0, l1);
      }
    }
    if (t == 0) (out + int64_t(rows) * width)[r] = 1.f / s;
  }
}

template <int LPR, int C4>
__global__ void __launch_bounds__(256) norm_bwd4_kernel(int rows, int width, float* __restrict__ in_adj, int64_t lda,
                                                        const float* __restrict__ out_adj, int64_t ldg,
                                                        const float* __restrict__ in, int64_t ldi,
                                                        const float* __restrict__ weight, int ln, int n_node,
                                                        float beta_node, float beta_edge,
                                                        const int* __restrict__ live_off) {
  constexpr int RPW = 64 / LPR;
  const int l = threadIdx.x & 63, t = l % LPR;
  const int r = (blockIdx.x * 4 + int(threadIdx.x >> 6)) * RPW + l / LPR;
  if (r >= rows) return;
  if (live_off && r >= n_node + live_off[n_node]) return;  // a capacity's dead row: no sink
  const float beta = r < n_node ? beta_node : beta_edge;
  const int w4 = width >> 2;
  const float4* x_row = reinterpret_cast<const float4*>(in + int64_t(r) * ldi);
  const float4* g_row = reinterpret_cast<const float4*>(out_adj + int64_t(r) * ldg);
  const float4* w4p = reinterpret_cast<const float4*>(weight);
  float4 x[C4], ga[C4], wq[C4];
#pragma unroll
  for (int j = 0; j < C4; ++j) {
    const int q = t + LPR * j;
    const bool in_range = q < w4;
    x[j] = in_range ? x_row[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    ga[j] = in_range ? g_row[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    wq[j] = in_range ? w4p[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mu = 0.0f;
  if (ln) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < C4; ++j) s += (x[j].x + x[j].y) + (x[j].z + x[j].w);
    mu = row_sum<LPR>(s) / width;
  }
  float sq = 0.0f, sg = 0.0f, sgx = 0.0f;
  auto acc1 = [&](float xv, float g, float w) {
    const float xc = xv - mu, gw = g * w;
    sq += xc * xc;
    sg += gw;
    sgx += gw * xc;
  };
#pragma unroll
  for (int j = 0; j < C4; ++j)
    if (t + LPR * j < w4) {  // a masked chunk's zeros would add mu^2 to the variance
      acc1(x[j].x, ga[j].x, wq[j].x), acc1(x[j].y, ga[j].y, wq[j].y);
      acc1(x[j].z, ga[j].z, wq[j].z), acc1(x[j].w, ga[j].w, wq[j].w);
    }
  sq = row_sum<LPR>(sq), sg = row_sum<LPR>(sg), sgx = row_sum<LPR>(sgx);
  const float inv = 1.0f / sqrtf(sq / width + (ln ? kLnEps : kRmsEps));
  const float mg = ln ? sg / width : 0.0f, mgx = sgx * inv / width;
  auto grad = [&](float xv, float g, float w) {
    const float a = fmaf(g, w, -mg), b = mul_rn(xv - mu, inv);
    return mul_rn(inv, fmaf(-b, mgx, a));
  };
  float4* a_row = reinterpret_cast<float4*>(in_adj + int64_t(r) * lda);
#pragma unroll
  for (int j = 0; j < C4; ++j) {
    const int q = t + LPR * j;
    if (q < w4) {
      float4 gq = make_float4(grad(x[j].x, ga[j].x, wq[j].x), grad(x[j].y, ga[j].y, wq[j].y),
                              grad(x[j].z, ga[j].z, wq[j].z), grad(x[j].w, ga[j].w, wq[j].w));
      if (beta != 0.0f) {
        const float4 o = a_row[q];
        gq = make_float4(beta * o.x + gq.x, beta * o.y + gq.y, beta * o.z + gq.z, beta * o.w + gq.w);
      }
      a_row[q] = gq;
    }
  }
}

template <int LPR, int C4>
__global__ void __launch_bounds__(256) rms_inv4_kernel(int rows, int width, const float* __restrict__ in, int64_t ldi,
                                                       float* __restrict__ inv) {
  constexpr int RPW = 64 / LPR;
  const int l = threadIdx.x & 63, t = l % LPR;
  const int r = (blockIdx.x * 4 + int(threadIdx.x >> 6)) * RPW + l / LPR;
  if (r >= rows) return;
  const int w4 = width >> 2;
  const float4* x_row = reinterpret_cast<const float4*>(in + int64_t(r) * ldi);
  float v = 0.0f;
#pragma unroll
  for (int j = 0; j < C4; ++j) {
    const int q = t + LPR * j;
    if (q < w4) {
      const float4 x = x_row[q];
      v += (x.x * x.x + x.y * x.y) + (x.z * x.z + x.w * x.w);
    }
  }
  v = row_sum<LPR>(v);
  if (t == 0) inv[r] = 1.0f / sqrtf(v / width + kRmsEps);
}

// f(lpr, c4) for a vectorisable width (a multiple of 4, <= 2048), rows a
// workgroup = 4 * 64 / lpr; -1 if the width does not vectorise.
template <class F>
int with_vec(int width, F&& f) {
  const int w4 = width / 4;
  if (width % 4 || w4 < 1 || w4 > 512) return -1;
  using std::integral_constant;
  if (w4 <= 16) return f(integral_constant<int, 16>{}, integral_constant<int, 1>{});
  if (w4 <= 32) return f(integral_constant<int, 32>{}, integral_constant<int, 1>{});
  if (w4 <= 64) return f(integral_constant<int, 64>{}, integral_constant<int, 1>{});
  if (w4 <= 128) return f(integral_constant<int, 64>{}, integral_constant<int, 2>{});
  if (w4 <= 256) return f(integral_constant<int, 64>{}, integral_constant<int, 4>{});
  return f(integral_constant<int, 64>{}, integral_constant<int, 8>{});
}
inline bool aligned16(const void* p, int64_t ld) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0;
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
  if (aligned16(in_adj, lda) && aligned16(out_adj, ldg) && aligned16(in, ldi) && aligned16(weight, 4)) {
    const int e = with_vec(width, [&](auto lc, auto cc) {
      constexpr int LPR = decltype(lc)::value, C4 = decltype(cc)::value, RPB = 4 * (64 / LPR);
      hipLaunchKernelGGL((norm_bwd4_kernel<LPR, C4>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, rows,
                         width, in_adj, lda, out_adj, ldg, in, ldi, weight, ln, n_node, beta_node, beta_edge,
                         live_off);
      return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
    });
    if (e >= 0) return e;
  }
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
  if (aligned16(in, ldi)) {
    const int e = with_vec(width, [&](auto lc, auto cc) {
      constexpr int LPR = decltype(lc)::value, C4 = decltype(cc)::value, RPB = 4 * (64 / LPR);
      hipLaunchKernelGGL((rms_inv4_kernel<LPR, C4>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, rows,
                         width, in, ldi, inv);
      return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
    });
    if (e >= 0) return e;
  }
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
  if (aligned16(out, ldo) && aligned16(in, ldi) && aligned16(weight, 4) && (!bias || aligned16(bias, 4))) {
    const int e = with_vec(width, [&](auto lc, auto cc) {
      constexpr int LPR = decltype(lc)::value, C4 = decltype(cc)::value, RPB = 4 * (64 / LPR);
      hipLaunchKernelGGL((norm_fwd4_kernel<LPR, C4>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st, rows,
                         width, out, ldo, in, ldi, weight, bias);
      return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
    });
    if (e >= 0) return e;
  }
  return with_lanes(width, [&](auto vc) {
    constexpr int V = decltype(vc)::value;
    hipLaunchKernelGGL(norm_fwd_kernel<V>, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, st, rows, width, out, ldo,
                       in, ldi, weight, bias);
    return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
  });
}

int pet_norm_rows_pairs(int rows, int width, void* out, const float* in, int64_t ldi, const float* weight,
                        const float* bias, void* stream) {
  if (rows < 0 || width < 8 || width % 8 || !out || !in || !weight || ldi < width) return PET_ATTN_EINVAL;
  if (rows == 0) return PET_ATTN_OK;
  if (!aligned16(out, 4) || !aligned16(in, ldi) || !aligned16(weight, 4) || (bias && !aligned16(bias, 4)))
    return PET_ATTN_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int e = with_vec(width, [&](auto lc, auto cc) {
    constexpr int LPR = decltype(lc)::value, C4 = decltype(cc)::value, RPB = 4 * (64 / LPR);
    hipLaunchKernelGGL((norm_fwd4_kernel<LPR, C4, true>), dim3(unsigned((rows + RPB - 1) / RPB)), dim3(256), 0, st,
                       rows, width, static_cast<float*>(out), int64_t(width), in, ldi, weight, bias);
    return hipGetLastError() == hipSuccess ? int(PET_ATTN_OK) : int(PET_ATTN_ELAUNCH);
  });
  return e >= 0 ? e : int(PET_ATTN_EINVAL);  // wider than the row kernels take
}

int pet_norm_rows_bwd(int rows, int width, float* in_adj, int64_t lda, float beta, const float* out_adj, int64_t ldg,
                      const float* in, int64_t ldi, const float* weight, int ln, void* stream) {
  return pet_rows_norm_bwd_sink(rows, width, in_adj, lda, out_adj, ldg, in, ldi, weight, ln, rows, beta, beta,
                                nullptr, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
