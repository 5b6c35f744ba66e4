// Dense layers on the fp32 matrix cores with the passes around them fused into
// the epilogue: C[M, N] = epi(A[M, K] B[N, K]^T), A and B row-major with K
// contiguous (torch Linear's in W^T; a backward in_adj = out_adj W uses W's
// transposed copy, so every GEMM has this one form).
//
// Epilogue, per element (i, j) in this order:
//   v = acc                                  (the product, fp32, fixed k order)
//   v = v * row_scale[i]                     (a row scale: RMSNorm's 1/rms, its weight folded into B)
//   v = v + bias[j]
//   v = v + beta * C_in[i, j]                (a residual, C_in may be C itself)
//   pre[i, j] = v                            (kept for a backward, when asked)
//   v = act(v)                               (SiLU, or SwiGLU on (v_2c, g_2c+1) pairs to column c)
// so the bias fills, residual sums and activation passes of the model need no
// memory round trip of their own.
//
// Tiling for gfx950: a 256-thread workgroup (4 waves in 2 x 2) computes a BM x BN
// tile, each wave (BM/2) x (BN/2) in 16 x 16 v_mfma_f32_16x16x4_f32 tiles. The
// K loop steps 16 at a time through LDS, double-buffered: each thread loads the
// next step's A and B slices into registers before the current step's MFMAs and
// stores them to the other buffer after, one barrier a step. Within a step the
// four MFMA k-slices take k = 4g + s (lane group g, slice s), so a lane reads
// one contiguous float4 of an A row and of a B row per 16 x 16 tile (the sum's
// order is fixed: results repeat bit for bit).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/pet_model.h"

namespace pet_gemm {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float sig_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

struct Epi {
  const float* row_scale = nullptr;  // [M]
  const float* bias = nullptr;       // [N]
  const float* cin = nullptr;        // [M, N] (ld ldcin), scaled by beta
  int64_t ldcin = 0;
  float beta = 0.f;
  float* pre = nullptr;              // [M, N] (ld ldpre): v before the activation
  int64_t ldpre = 0;
  int act = 0;                       // 0 none, 1 SiLU, 2 SwiGLU (C has N/2 columns)
};

template <int BM, int BN, int BK = 32>
__global__ void __launch_bounds__(256) gemm_nt_kernel(int M, int N, int K, const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb, float* C, int64_t ldc,
                                                      Epi epi) {
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16, PK = BK + 4, Q4 = BK / 4;
  // float4 slots of a step's A / B slice (4 a row), and a thread's share
  constexpr int AQ = BM * BK / 4, BQ = BN * BK / 4, AL = (AQ + 255) / 256, BL = (BQ + 255) / 256;
  __shared__ float As[2][BM * PK], Bs[2][BN * PK];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w >> 1, wn = w & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  f4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

  // thread t loads float4 slots q = t + 256 u: row q / 4, columns 4 (q % 4) ..
  float4 ra[AL], rb[BL];
  auto load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < AL; ++u) {
      const int q = tid + 256 * u, r = q / Q4, i = m0 + r;
      ra[u] = q < AQ && i < M ? *reinterpret_cast<const float4*>(A + int64_t(i) * lda + k0 + 4 * (q % Q4))
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      const int q = tid + 256 * u, r = q / Q4, j = n0 + r;
      rb[u] = q < BQ && j < N ? *reinterpret_cast<const float4*>(B + int64_t(j) * ldb + k0 + 4 * (q % Q4))
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < AL; ++u) {
      const int q = tid + 256 * u;
      if (q < AQ) *reinterpret_cast<float4*>(&As[buf][(q / Q4) * PK + 4 * (q % Q4)]) = ra[u];
    }
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      const int q = tid + 256 * u;
      if (q < BQ) *reinterpret_cast<float4*>(&Bs[buf][(q / Q4) * PK + 4 * (q % Q4)]) = rb[u];
    }
  };

  const int steps = K / BK;  // K a multiple of BK
  load(0);
  store(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int cur = s & 1;
    if (s + 1 < steps) load((s + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {  // 16 k a sub-step: k = kk + 4g + slice
      float4 av[TM], bv[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a)
        av[a] = *reinterpret_cast<const float4*>(&As[cur][(wm * WM + 16 * a + c) * PK + kk + 4 * g]);
#pragma unroll
      for (int b = 0; b < TN; ++b)
        bv[b] = *reinterpret_cast<const float4*>(&Bs[cur][(wn * WN + 16 * b + c) * PK + kk + 4 * g]);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) {
          acc[a][b] = mfma(av[a].x, bv[b].x, acc[a][b]);
          acc[a][b] = mfma(av[a].y, bv[b].y, acc[a][b]);
          acc[a][b] = mfma(av[a].z, bv[b].z, acc[a][b]);
          acc[a][b] = mfma(av[a].w, bv[b].w, acc[a][b]);
        }
    }
    if (s + 1 < steps) {
      store(cur ^ 1);
      __syncthreads();
    }
  }

  // epilogue: lane (c, g) of tile (a, b) holds rows 4g + r, column c
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int j = n0 + wn * WN + 16 * b + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = m0 + wm * WM + 16 * a + 4 * g + r;
        float v = acc[a][b][r];
        if (epi.row_scale && i < M) v *= epi.row_scale[i];
        if (epi.bias && j < N) v += epi.bias[j];
        if (epi.cin && i < M && j < N) v += epi.beta * epi.cin[int64_t(i) * epi.ldcin + j];
        if (epi.pre && i < M && j < N) epi.pre[int64_t(i) * epi.ldpre + j] = v;
        if (epi.act == 2) {
          // SwiGLU: columns 2c' (value) and 2c'+1 (gate) sit in lanes c and c + 1
          const float gate = __shfl_down(v, 1, 16);
          if ((c & 1) == 0 && i < M && j < N) C[int64_t(i) * ldc + j / 2] = v * sig_fast(gate);
        } else if (i < M && j < N) {
          C[int64_t(i) * ldc + j] = epi.act == 1 ? v * sig_fast(v) : v;
        }
      }
    }
}

}  // namespace pet_gemm

using namespace pet_gemm;

// The tile shape for a problem: wide outputs take 128 x 128; narrow ones
// (N <= 64) or too few tiles to fill 256 CUs take smaller tiles.
int pet_gemm_nt_fused(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta, float* pre,
                int64_t ldpre, int act, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (K % 16 || lda % 4 || ldb % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(B) & 15))
    return PET_ATTN_EALIGN;
  if (act == 2 && N % 2) return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  auto tiles = [&](int bm, int bn) { return int64_t((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  const bool k32 = K % 32 == 0;
  auto go = [&](auto kern, int bm, int bn) {
    hipLaunchKernelGGL(kern, dim3(unsigned((N + bn - 1) / bn), unsigned((M + bm - 1) / bm)), dim3(256), 0, st, M, N,
                       K, A, lda, B, ldb, C, ldc, e);
  };
  if (N > 64 && tiles(128, 128) >= 512)
    k32 ? go(gemm_nt_kernel<128, 128, 32>, 128, 128) : go(gemm_nt_kernel<128, 128, 16>, 128, 128);
  else if (N > 32 && tiles(128, 64) >= 512)
    k32 ? go(gemm_nt_kernel<128, 64, 32>, 128, 64) : go(gemm_nt_kernel<128, 64, 16>, 128, 64);
  else
    k32 ? go(gemm_nt_kernel<64, 32, 32>, 64, 32) : go(gemm_nt_kernel<64, 32, 16>, 64, 32);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

extern "C" int pet_linear_fused(int M, int N, int K, const float* A, int64_t lda, const float* W, int64_t ldw,
                                float* C, int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!A || !W || !C || ldc < (act == 2 ? N / 2 : N) || lda < K || ldw < K ||
                           (cin && ldcin < N) || (pre && ldpre < N) || act < 0 || act > 2))
    return PET_ATTN_EINVAL;
  return pet_gemm_nt_fused(M, N, K, A, lda, W, ldw, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre, act,
                           reinterpret_cast<hipStream_t>(stream));
}
