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

#include <algorithm>
#include <cstdint>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <cstdlib>

#include "../../include/pet_model.h"
#include "split_bf16.h"

namespace pet_gemm {

using pet_split::f4;
using pet_split::mfma6;
using pet_split::pack_hi;
using pet_split::split3;
using pet_split::split8;
using pet_split::u4;
using pet_split::u2;
using pet_split::mfma3;
using pet_split::mfma_h;
using pet_split::pair2;
using pet_split::pair_scale;

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
  int act = 0;                       // 0 none, 1 SiLU, 2 SwiGLU (C has N/2 columns),
                                     // 3 / 4 the backward of SiLU / SwiGLU (below)
  // Block pairs in place of C (staged epilogue only): the output row i as
  // fp16 pairs in pair_act_kernel's layout (kgo k groups of 8 a row, each
  // group's hi then lo 16 bytes), scaled per (row, column tile) -- the tile's
  // output columns are one K block of the product that reads them -- with the
  // block's inverse scale at pinv[block ldinv + i].
  u4* pout = nullptr;
  float* pinv = nullptr;
  int64_t ldinv = 0;
  int kgo = 0;
};

// FLOPs (2 M N K) of the products this library's dense kernels have launched,
// by the instructions that run them: 0 the fp32 fused kernel (fp32 matrix
// cores), 1 split-fp32 as three bf16 parts (six bf16 products), 2 fp16 pairs
// (three fp16 products), 3 the short-K kernel (five fp16 products). A
// measurement aid, process-wide (pet_gemm_flop_tally).
std::atomic<uint64_t> g_flops[4];
inline void tally(int cls, int64_t M, int64_t N, int64_t K) {
  g_flops[cls].fetch_add(uint64_t(2) * uint64_t(M) * uint64_t(N) * uint64_t(K), std::memory_order_relaxed);
}

// The epilogue of one result element v at (i, j), shared by the kernels. Every
// lane of the wave calls it together (SwiGLU pairs neighbouring lanes):
// (i, j) may lie outside the result, which is then left alone.
__device__ __forceinline__ void epi_elem(float v, int i, int j, int c, int M, int N, float* C, int64_t ldc,
                                         const Epi& epi) {
  if (epi.act >= 3) {
    // v is an activation's output adjoint; cin the saved pre-activation
    // (bias the pre-activation's bias, null when cin holds it already).
    // 3: C[i, j] = v silu'(z); 4 (SwiGLU, (value, gate) pairs of cin):
    // C[i, 2j] = v sigmoid(g), C[i, 2j + 1] = v u sigmoid(g) (1 - sigmoid(g))
    if (i >= M || j >= N) return;
    const float* z = epi.cin + int64_t(i) * epi.ldcin;
    if (epi.act == 3) {
      const float x = z[j] + (epi.bias ? epi.bias[j] : 0.f), sg = sig_fast(x);
      C[int64_t(i) * ldc + j] = v * (sg * (1.0f + x * (1.0f - sg)));
    } else {
      const float u = z[2 * j] + (epi.bias ? epi.bias[2 * j] : 0.f);
      const float sg = sig_fast(z[2 * j + 1] + (epi.bias ? epi.bias[2 * j + 1] : 0.f));
      *reinterpret_cast<float2*>(C + int64_t(i) * ldc + 2 * j) = make_float2(v * sg, v * u * sg * (1.0f - sg));
    }
    return;
  }
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
// The tile kernels' epilogue: lane (c, g) of tile (a, b) holds rows 4g + r,
// column c of the wave's WM x WN share.
template <int WM, int WN>
__device__ __forceinline__ void epilogue(const f4 (&acc)[WM / 16][WN / 16], int m0, int n0, int wm, int wn, int c,
                                         int g, int M, int N, float* C, int64_t ldc, const Epi& epi) {
  constexpr int TM = WM / 16, TN = WN / 16;
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        epi_elem(acc[a][b][r], m0 + wm * WM + 16 * a + 4 * g + r, n0 + wn * WN + 16 * b + c, c, M, N, C, ldc, epi);
}

// The epilogue through LDS, for a tile whose columns all lie in the result:
// the waves' results (already unscaled) go to a BM x BN fp32 tile in LDS
// (float4 slot q of row R at q ^ s(R), s(R) = 4 (R / 4) mod BN / 4, so the
// four row groups of a store fall on distinct banks), then each thread takes
// float4 runs of a row and applies epi_elem's arithmetic, in its order, with
// 16-byte loads and stores (C, pre, cin, bias) in place of a wave's 4-byte
// stores to four rows. False (nothing written) where a pointer or leading
// dimension does not allow the 16-byte accesses; the caller then uses
// epilogue(). tile: BM BN floats of LDS no wave still reads.
template <int BM, int BN, int WGM, int WGN, int PASSES = 1, bool PO = false>
__device__ __forceinline__ bool staged_epilogue(const f4 (&acc)[BM / WGM / 16][BN / WGN / 16], float* tile, int m0,
                                                int n0, int M, int N, float* C, int64_t ldc, const Epi& epi) {
  constexpr int T = 64 * WGM * WGN, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16, F = BN / 4;
  constexpr int RB = BM / PASSES;  // the tile's rows a pass (the rows of WGM / PASSES wave rows)
  static_assert(T % F == 0 && WGM % PASSES == 0, "whole rows a pass, whole wave rows a pass");
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool act4 = epi.act == 4, act2 = epi.act == 2;
  // C's columns: 2 N (act 4), N / 2 (act 2), else N; j stays a multiple of 4
  const bool ok = n0 + BN <= N && (PO || (a16(C) && ldc % 4 == 0)) && (!epi.bias || a16(epi.bias)) &&
                  (!epi.cin || (a16(epi.cin) && epi.ldcin % 4 == 0)) && (!epi.pre || (a16(epi.pre) && epi.ldpre % 4 == 0));
  if (!ok) return false;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w / WGN, wn = w % WGN;
  auto slot = [](int R, int q) { return R * BN + 4 * (q ^ ((4 * (R >> 2)) & (F - 1))); };
  const int q = tid % F;
  const int j = n0 + 4 * q;
  // a thread's NO outputs of row i from output column jo on: to C, or (block
  // pairs) split by the power of two that puts the largest |output| of the
  // row's BN-column tile at [2^14, 2^15) -- the row's F threads are
  // consecutive lanes, F 16 or 32 -- with one thread a row writing the
  // inverse scale
  auto put = [&](int i, int jo, const float* o, auto no_c) {
    constexpr int NO = decltype(no_c)::value;
    if constexpr (!PO) {
      float* dst = C + int64_t(i) * ldc + jo;
      if constexpr (NO == 2) *reinterpret_cast<float2*>(dst) = make_float2(o[0], o[1]);
      if constexpr (NO >= 4) *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      if constexpr (NO == 8) *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
    } else {
    static_assert(F == 16 || F == 32, "a row's threads one or two DPP rows");
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < NO; ++e) m = fmaxf(m, fabsf(o[e]));
    int mb = __float_as_int(m);  // |values|: the bit patterns order as the values
#define PET_ROR(n) mb = max(mb, __builtin_amdgcn_update_dpp(0, mb, 0x120 + (n), 0xf, 0xf, true))
    PET_ROR(1);
    PET_ROR(2);
    PET_ROR(4);
    PET_ROR(8);
#undef PET_ROR
    if constexpr (F == 32) mb = max(mb, __shfl_xor(mb, 16));
    const float sc = pair_scale(__int_as_float(mb));
    unsigned h[NO / 2], lw[NO / 2];
#pragma unroll
    for (int e = 0; e < NO / 2; ++e) pair2(o[2 * e] * sc, o[2 * e + 1] * sc, h[e], lw[e]);
    unsigned* hi = reinterpret_cast<unsigned*>(epi.pout + (int64_t(i) * epi.kgo + jo / 8) * 2) + (jo % 8) / 2;
    if constexpr (NO == 2) hi[0] = h[0], hi[4] = lw[0];
    if constexpr (NO == 4) {
      *reinterpret_cast<u2*>(hi) = u2{h[0], h[1]};
      *reinterpret_cast<u2*>(hi + 4) = u2{lw[0], lw[1]};
    }
    if constexpr (NO == 8) {
      *reinterpret_cast<u4*>(hi) = u4{h[0], h[1], h[2], h[3]};
      *reinterpret_cast<u4*>(hi + 4) = u4{lw[0], lw[1], lw[2], lw[3]};
    }
    if (q == 0) epi.pinv[int64_t(n0 / BN) * epi.ldinv + i] = 1.f / sc;
    }
  };
  using c2 = std::integral_constant<int, 2>;
  using c4 = std::integral_constant<int, 4>;
  using c8 = std::integral_constant<int, 8>;
  float4 bj = make_float4(0.f, 0.f, 0.f, 0.f), bj2 = bj;
  if (epi.bias) {
    if (act4) {
      bj = *reinterpret_cast<const float4*>(epi.bias + 2 * j);
      bj2 = *reinterpret_cast<const float4*>(epi.bias + 2 * j + 4);
    } else {
      bj = *reinterpret_cast<const float4*>(epi.bias + j);
    }
  }
  for (int h = 0; h < PASSES; ++h) {
  __syncthreads();  // every wave done with the LDS the tile reuses
  if (wm / (WGM / PASSES) == h) {
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int R = wm * WM + 16 * a + 4 * g + rr - h * RB, Cc = wn * WN + 16 * b + c;
          tile[slot(R, Cc >> 2) + (Cc & 3)] = acc[a][b][rr];
        }
  }
  __syncthreads();
  for (int R = tid / F; R < RB; R += T / F) {
    const int i = m0 + h * RB + R;
    if (i >= M) break;
    const float4 t4 = *reinterpret_cast<const float4*>(tile + slot(R, q));
    float v[4] = {t4.x, t4.y, t4.z, t4.w};
    if (epi.act >= 3) {
      const float* z = epi.cin + int64_t(i) * epi.ldcin;
      if (!act4) {
        const float4 z4 = *reinterpret_cast<const float4*>(z + j);
        const float zz[4] = {z4.x, z4.y, z4.z, z4.w}, bb[4] = {bj.x, bj.y, bj.z, bj.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = zz[e] + (epi.bias ? bb[e] : 0.f), sg = sig_fast(x);
          o[e] = v[e] * (sg * (1.0f + x * (1.0f - sg)));
        }
        put(i, j, o, c4{});
      } else {
        const float4 z0 = *reinterpret_cast<const float4*>(z + 2 * j), z1 = *reinterpret_cast<const float4*>(z + 2 * j + 4);
        const float zz[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
        const float bb[8] = {bj.x, bj.y, bj.z, bj.w, bj2.x, bj2.y, bj2.z, bj2.w};
        float o[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = zz[2 * e] + (epi.bias ? bb[2 * e] : 0.f);
          const float sg = sig_fast(zz[2 * e + 1] + (epi.bias ? bb[2 * e + 1] : 0.f));
          o[2 * e] = v[e] * sg, o[2 * e + 1] = v[e] * u * sg * (1.0f - sg);
        }
        put(i, 2 * j, o, c8{});
      }
      continue;
    }
    if (epi.row_scale) {
      const float rs = epi.row_scale[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] *= rs;
    }
    if (epi.bias) v[0] += bj.x, v[1] += bj.y, v[2] += bj.z, v[3] += bj.w;
    if (epi.cin) {
      const float4 c4 = *reinterpret_cast<const float4*>(epi.cin + int64_t(i) * epi.ldcin + j);
      v[0] += epi.beta * c4.x, v[1] += epi.beta * c4.y, v[2] += epi.beta * c4.z, v[3] += epi.beta * c4.w;
    }
    if (epi.pre) *reinterpret_cast<float4*>(epi.pre + int64_t(i) * epi.ldpre + j) = make_float4(v[0], v[1], v[2], v[3]);
    if (act2) {
      const float o[2] = {v[0] * sig_fast(v[1]), v[2] * sig_fast(v[3])};
      put(i, j / 2, o, c2{});
    } else {
      if (epi.act == 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] * sig_fast(v[e]);
      put(i, j, v, c4{});
    }
  }
  }
  return true;
}

template <int BM, int BN, int BK = 32>
__global__ void __launch_bounds__(256) gemm_nt_kernel(int M, int N, int K, const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb, float* C, int64_t ldc,
                                                      Epi epi) {
  constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16, PK = BK + 4, Q4 = BK / 4;
  // float4 slots of a step's A / B slice (4 a row), and a thread's share
  constexpr int AQ = BM * BK / 4, BQ = BN * BK / 4, AL = (AQ + 255) / 256, BL = (BQ + 255) / 256;
  __shared__ float lds_ab[2 * (BM + BN) * PK];  // both buffers of A's and B's slices, one array
  float (*const As)[BM * PK] = reinterpret_cast<float (*)[BM * PK]>(lds_ab);
  float (*const Bs)[BN * PK] = reinterpret_cast<float (*)[BN * PK]>(lds_ab + 2 * BM * PK);
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w >> 1, wn = w & 1;
  // a 1-D grid of tiles, a row block's column tiles consecutive
  const int NT = (N + BN - 1) / BN, tile = blockIdx.x;
  const int m0 = (tile / NT) * BM, n0 = (tile % NT) * BN;

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
  // through LDS (both slice buffers, done with), a pass per wave row
  static_assert((BM / 2) * BN <= 2 * (BM + BN) * PK, "a wave row's results fit the slices' LDS");
  if (!staged_epilogue<BM, BN, 2, 2, 2>(acc, &As[0][0], m0, n0, M, N, C, ldc, epi))
    epilogue<WM, WN>(acc, m0, n0, wm, wn, c, g, M, N, C, ldc, epi);
}

// The same product with the fp32 matrix cores' work moved to the bf16 ones:
// B comes split once (pet_linear_split_weights: per row, per 8-element k
// group, its three bf16 parts, 48 bytes), A is split as each k step of 32 is
// staged, and a 16 x 16 x 32 step is the six part products of split_bf16.h
// (6 x 16 nominal cycles against 8 x 32 on the fp32 instruction, at fp32's
// error; measured with all waves issuing, ~33 against ~42 cycles an instruction).
// Tiles of WGM x WGN waves (64 WGM WGN threads): 64 x 64 or 128 x 64 of 2 x 2,
// 128 x 128 of 2 x 4. K steps of 32 go through one LDS buffer, the next
// step's slices loaded into registers under the current step's products. A
// row's step is 4 groups x 3 parts x 16 bytes plus a 32-byte pad (14 u4: the
// 8-byte stores of an A slice's neighbouring rows then fall on distinct banks,
// while the 128-bit operand reads stay conflict-free; measured 3-4% faster
// than a 16-byte pad at the model's large shapes, 131072 x 1536 x 512 1160
// against 1208 us): 28 / 42 / 56 KB a workgroup. K a multiple of 32.
// Measured against torch's GEMM at the model's shapes: even at K = 128
// (27318 x 128 x 128: 15 against 20 us), ahead at 26670 x 1024 x 128 (59-62
// against 86 us) and 131072 x 1536 x 512 (1160 against 1555 us); rocBLAS's
// fp32 kernel takes 12.8 us on the first.
//
// BF: B comes as fp32 rows [N, K] (ld ldb) and is split as it is staged, like
// A (for a caller with no room to keep a split copy: twice the staging VALU).
template <int BM, int BN, int WGM = 2, int WGN = 2, bool BF = false>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_nt_split_kernel(int M, int N, int K,
                                                                       const float* __restrict__ A, int64_t lda,
                                                                       const u4* __restrict__ Bs, float* C,
                                                                       int64_t ldc, Epi epi,
                                                                       const float* __restrict__ Bf, int64_t ldb,
                                                                       int /* one tile an item */) {
  constexpr int T = 64 * WGM * WGN, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16, RP = 14;
  constexpr int AQ = BM * 8, AL = (AQ + T - 1) / T;   // float4 of a step's A slice, a thread's share
  constexpr int BQ = BF ? BN * 8 : BN * 12, BL = (BQ + T - 1) / T;  // B slice: float4 (BF) or u4 slots
  __shared__ u4 lds_ab[(BM + BN) * RP];  // A's and B's step slices, one array (the epilogue's tile spans both)
  u4* const As = lds_ab;
  u4* const Bt = lds_ab + BM * RP;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w / WGN, wn = w % WGN;
  // Workgroups go to the 8 XCDs in turn (an L2 each): XCD k takes a
  // contiguous run of tiles in row-block order, so a row block's column tiles
  // share an L2 (509730 x 512 x 512: 1547 against 1624 us in launch order).
  // A bijection of the tiles whatever the hardware's order.
  // A 1-D grid of all the tiles, tile t = (row block t / NT, column tile t % NT).
  const int NT = (N + BN - 1) / BN, total = gridDim.x, L = blockIdx.x;
  const int q = total / 8, r = total % 8, x = L % 8;
  const int t = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + L / 8;
  const int tm = t / NT, tn = t % NT;
  const int m0 = tm * BM, n0 = tn * BN, KG = K / 8;

  f4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

  // A: thread t's float4 slots q = t + 256 u, row q / 8, k 4 (q % 8) .. ;
  // B: u4 slots q, row q / 12, part (q % 12) of the row's step
  float4 ra[AL];
  u4 rb[BF ? 1 : BL];
  float4 rbf[BF ? BL : 1];
  auto load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < AL; ++u) {
      const int q = tid + T * u, i = m0 + q / 8;
      ra[u] = q < AQ && i < M ? *reinterpret_cast<const float4*>(A + int64_t(i) * lda + k0 + 4 * (q % 8))
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      if constexpr (BF) {
        const int q = tid + T * u, j = n0 + q / 8;
        rbf[u] = q < BQ && j < N ? *reinterpret_cast<const float4*>(Bf + int64_t(j) * ldb + k0 + 4 * (q % 8))
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const int q = tid + T * u, j = n0 + q / 12;
        rb[u] = q < BQ && j < N ? Bs[(int64_t(j) * KG + k0 / 8) * 3 + q % 12] : u4{0u, 0u, 0u, 0u};
      }
    }
  };
  // a float4 of row `row`'s k slots 4 (q % 8) .. into its split row (parts of
  // k group (q % 8) / 2, half q & 1) of tile X
  auto store_split = [&](u4* X, int row, int q, const float4& v) {
    float h[3][4];
    split3(v.x, h[0][0], h[1][0], h[2][0]);
    split3(v.y, h[0][1], h[1][1], h[2][1]);
    split3(v.z, h[0][2], h[1][2], h[2][2]);
    split3(v.w, h[0][3], h[1][3], h[2][3]);
    unsigned* dst = reinterpret_cast<unsigned*>(&X[row * RP + ((q % 8) / 2) * 3]) + 2 * (q & 1);
#pragma unroll
    for (int p = 0; p < 3; ++p)
      *reinterpret_cast<uint2*>(dst + 4 * p) = make_uint2(pack_hi(h[p][0], h[p][1]), pack_hi(h[p][2], h[p][3]));
  };
  auto store = [&]() {
#pragma unroll
    for (int u = 0; u < AL; ++u) {
      // the float4 is half of k group (q % 8) / 2: its parts go to that half of each part's 16 bytes
      const int q = tid + T * u;
      if (q < AQ) store_split(As, q / 8, q, ra[u]);
    }
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      const int q = tid + T * u;
      if constexpr (BF) {
        if (q < BQ) store_split(Bt, q / 8, q, rbf[u]);
      } else {
        if (q < BQ) Bt[(q / 12) * RP + q % 12] = rb[u];
      }
    }
  };

  const int steps = K / 32;
  load(0);
  store();
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    if (s + 1 < steps) load((s + 1) * 32);
    u4 av[TM][3], bv[TN][3];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int p = 0; p < 3; ++p) av[a][p] = As[(wm * WM + 16 * a + c) * RP + 3 * g + p];
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int p = 0; p < 3; ++p) bv[b][p] = Bt[(wn * WN + 16 * b + c) * RP + 3 * g + p];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) acc[a][b] = mfma6(av[a], bv[b], acc[a][b]);
    if (s + 1 < steps) {
      __syncthreads();  // every wave is done with the step's slices
      store();
      __syncthreads();
    }
  }
  // through LDS (the slices', done with), a pass per wave row
  static_assert((BM / WGM) * BN * 4 <= (BM + BN) * RP * 16, "a wave row's results fit the slices' LDS");
  if (!staged_epilogue<BM, BN, WGM, WGN, WGM>(acc, reinterpret_cast<float*>(lds_ab), m0, n0, M, N, C, ldc, epi))
    epilogue<WM, WN>(acc, m0, n0, wm, wn, c, g, M, N, C, ldc, epi);
}

// W^T as split rows, W [K, N] (ld ldw): out[(n K/8 + j) 3 + p] = part p of
// column n's k group j.
__global__ void split_rows_t_kernel(const float* __restrict__ W, int N, int K, int64_t ldw, u4* __restrict__ out) {
  const int KG = K / 8;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= int64_t(N) * KG) return;
  const int n = int(t % N), j = int(t / N);  // consecutive threads, consecutive columns of a row
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = W[int64_t(8 * j + e) * ldw + n];
  u4 parts[3];
  split8(x, parts);
#pragma unroll
  for (int p = 0; p < 3; ++p) out[(int64_t(n) * KG + j) * 3 + p] = parts[p];
}

// W [N, K] (ld ldw) as split rows: out[(n K/8 + j) 3 + p] = part p of k group j.
__global__ void split_rows_kernel(const float* __restrict__ W, int N, int K, int64_t ldw, u4* __restrict__ out) {
  const int KG = K / 8;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= int64_t(N) * KG) return;
  const int n = int(t / KG), j = int(t % KG);
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = W[int64_t(n) * ldw + 8 * j + e];
  u4 parts[3];
  split8(x, parts);
#pragma unroll
  for (int p = 0; p < 3; ++p) out[t * 3 + p] = parts[p];
}

// C = epi(A B^T) with B as fp16 pairs made once (pair_rows_kernel:
// per row, per 8-element k group, its hi and lo parts, 32 bytes, then the
// rows' inverse scales) and A split as each k step of 32 is staged, after a
// first pass over the tile's rows for their scales. Tiles of WGM x WGN waves
// (64 WGM WGN threads): 64 x 64 or 128 x 64 of 2 x 2, 128 x 128 of 2 x 4. K
// steps of 32 go through one LDS buffer, the next step's slices loaded into
// registers under the current step's products. A row's step is 4 groups x 2
// parts x 16 bytes plus a 16-byte pad (9 u4: 16 consecutive rows' 128-bit
// operand reads fall on distinct banks). K a multiple of 32.
//
// BF: B comes as fp32 rows [N, K] (ld ldb) and is split as it is staged, like
// A (for a caller with no room to keep a split copy), its row scales from the
// same first pass.
template <int BM, int BN, int WGM = 2, int WGN = 2, bool BF = false>
__global__ void __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(BN == 128 ? 4 : BM == 128 ? 2 : 3))) gemm_nt_pair_kernel(int M, int N, int K,
                                                                       const float* __restrict__ A, int64_t lda,
                                                                       const u4* __restrict__ Bs, float* C,
                                                                       int64_t ldc, Epi epi,
                                                                       const float* __restrict__ Bf, int64_t ldb,
                                                                       int cpw) {
  constexpr int T = 64 * WGM * WGN, NW = T / 64, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16, RP = 9;
  constexpr int AL = BM * 8 / T;  // float4 of a step's A slice, a thread's share
  constexpr int BL = BN * 8 / T;  // B slice: float4 (BF) or u4 slots, a thread's share
  static_assert(AL * T == BM * 8 && BL * T == BN * 8, "a step's slices divide evenly over the threads");
  __shared__ u4 lds_ab[(BM + BN) * RP];  // A's and B's step slices, one array (the epilogue's tile spans both)
  u4* const As = lds_ab;
  u4* const Bt = lds_ab + BM * RP;
  __shared__ float sa[BM], sb[BF ? BN : 1];  // row scales of the tile's A rows (and B rows with BF)
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w / WGN, wn = w % WGN;
  // Workgroups go to the 8 XCDs in turn (an L2 each): XCD k takes a
  // contiguous run of tiles in row-block order, so a row block's column tiles
  // share an L2 (509730 x 512 x 512: 1547 against 1624 us in launch order).
  // A bijection of the tiles whatever the hardware's order.
  // A 1-D grid of work items, item t = (row block t / NG, its column tiles
  // cpw (t % NG) .. in turn): the A rows' scales are found once for cpw tiles.
  const int NT = (N + BN - 1) / BN, NG = (NT + cpw - 1) / cpw, total = gridDim.x, L = blockIdx.x;
  const int q = total / 8, r = total % 8, x = L % 8;
  const int t = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + L / 8;
  const int tm = t / NG, tn0 = (t % NG) * cpw, tn1 = min(tn0 + cpw, NT);
  const int m0 = tm * BM, KG = K / 8;
  int n0 = tn0 * BN;

  // The first pass: wave w takes rows w, w + NW, ..., a float4 a lane along
  // k, all its rows' loads in flight together, then each row's largest |x|
  // reduced over the wave. Rows past M (N) read the last row: their results
  // are never stored.
  auto row_scales = [&](const float* X, int64_t ldx, int rows, auto nr, float* s) {
    constexpr int RW = decltype(nr)::value / NW, RB = RW < 8 ? RW : 8;  // rows a wave, a batch
#pragma unroll
    for (int j0 = 0; j0 < RW; j0 += RB) {
      unsigned o[RB];  // row offsets from X (a tile's rows: within 2^32 floats)
      float m[RB];
#pragma unroll
      for (int j = 0; j < RB; ++j) o[j] = unsigned(min(w + NW * (j0 + j), rows - 1)) * unsigned(ldx), m[j] = 0.f;
      for (int k = 4 * l; k < K; k += 256) {
        float4 v[RB];
#pragma unroll
        for (int j = 0; j < RB; ++j) v[j] = *reinterpret_cast<const float4*>(X + o[j] + k);
#pragma unroll
        for (int j = 0; j < RB; ++j)
          m[j] = fmaxf(m[j], fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
      }
#pragma unroll
      for (int j = 0; j < RB; ++j) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m[j] = fmaxf(m[j], __shfl_xor(m[j], o));
        if (l == 0) s[w + NW * (j0 + j)] = pair_scale(m[j]);
      }
    }
  };
  row_scales(A + int64_t(m0) * lda, lda, M - m0, std::integral_constant<int, BM>(), sa);
  __syncthreads();

  // A: thread t's float4 slots q = t + T u, row q / 8, k 4 (q % 8) .. ;
  // B: u4 slots q, row q / 8, part (q % 8) of the row's step
  float4 ra[AL];
  float rsa[AL];
  u4 rb[BF ? 1 : BL];
  float4 rbf[BF ? BL : 1];
  float rsb[BF ? BL : 1];
  const float* pa[AL];
#pragma unroll
  for (int u = 0; u < AL; ++u) {
    const int qq = tid + T * u;
    pa[u] = A + int64_t(min(m0 + qq / 8, M - 1)) * lda + 4 * (qq % 8);
    rsa[u] = sa[qq / 8];
  }
  auto load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < AL; ++u) ra[u] = *reinterpret_cast<const float4*>(pa[u] + k0);
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      const int qq = tid + T * u, j = min(n0 + qq / 8, N - 1);
      if constexpr (BF)
        rbf[u] = *reinterpret_cast<const float4*>(Bf + int64_t(j) * ldb + k0 + 4 * (qq % 8));
      else
        rb[u] = Bs[(int64_t(j) * KG + k0 / 8) * 2 + qq % 8];
    }
  };
  // a float4 of row `row`'s k slots 4 (q % 8) .. , scaled by s, into its
  // row's hi and lo parts of k group (q % 8) / 2, half q & 1, of tile X
  auto store_pair = [&](u4* X, int row, int qq, const float4& v, float s) {
    unsigned h0, l0, h1, l1;
    pair2(v.x * s, v.y * s, h0, l0);
    pair2(v.z * s, v.w * s, h1, l1);
    unsigned* dst = reinterpret_cast<unsigned*>(&X[row * RP + ((qq % 8) / 2) * 2]) + 2 * (qq & 1);
    *reinterpret_cast<uint2*>(dst) = make_uint2(h0, h1);
    *reinterpret_cast<uint2*>(dst + 4) = make_uint2(l0, l1);
  };
  auto store = [&]() {
#pragma unroll
    for (int u = 0; u < AL; ++u) {
      const int qq = tid + T * u;
      store_pair(As, qq / 8, qq, ra[u], rsa[u]);
    }
#pragma unroll
    for (int u = 0; u < BL; ++u) {
      const int qq = tid + T * u;
      if constexpr (BF)
        store_pair(Bt, qq / 8, qq, rbf[u], rsb[u]);
      else
        Bt[(qq / 8) * RP + qq % 8] = rb[u];
    }
  };

  const int steps = K / 32;
  for (int tn = tn0; tn < tn1; ++tn) {
  n0 = tn * BN;
  if constexpr (BF) {
    row_scales(Bf + int64_t(n0) * ldb, ldb, N - n0, std::integral_constant<int, BN>(), sb);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < BL; ++u) rsb[u] = sb[(tid + T * u) / 8];
  }
  f4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
  load(0);
  store();
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    if (s + 1 < steps) load((s + 1) * 32);
    u4 av[TM][2], bv[TN][2];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int p = 0; p < 2; ++p) av[a][p] = As[(wm * WM + 16 * a + c) * RP + 2 * g + p];
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int p = 0; p < 2; ++p) bv[b][p] = Bt[(wn * WN + 16 * b + c) * RP + 2 * g + p];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) acc[a][b] = mfma3(av[a], bv[b], acc[a][b]);
    if (s + 1 < steps) {
      __syncthreads();  // every wave is done with the step's slices
      store();
      __syncthreads();
    }
  }
  // the scales undone: rows 4g + r of each 16-row block (from LDS), this
  // lane's columns (from the split weights' inverse scales, or LDS with BF)
  const float* inv_b = reinterpret_cast<const float*>(Bs + int64_t(N) * KG * 2);
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int jj = wn * WN + 16 * b + c;
    const float ib = BF ? 1.f / sb[jj] : inv_b[min(n0 + jj, N - 1)];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) acc[a][b][rr] = acc[a][b][rr] * (1.f / sa[wm * WM + 16 * a + 4 * g + rr]) * ib;
  }
  // (m0 laundered per tile: the epilogue's row addresses are then made
  // here, not hoisted out of the tile loop into registers held across it)
  int m0t = m0;
  asm volatile("" : "+s"(m0t));
  // through LDS (As and Bt, done with), a pass per wave row
  static_assert((BM / WGM) * BN * 4 <= (BM + BN) * RP * 16, "a wave row's results fit the slices' LDS");
  if (!staged_epilogue<BM, BN, WGM, WGN, WGM>(acc, reinterpret_cast<float*>(As), m0t, n0, M, N, C, ldc, epi))
    epilogue<WM, WN>(acc, m0t, n0, wm, wn, c, g, M, N, C, ldc, epi);
  __syncthreads();  // the next tile's first slices overwrite this one's last
  }
}

// Rows of B = W (transposed false: W [N, K], ld ldw) or B = W^T (transposed
// true: W [K, N]) as P fp16 parts: out[(n K/8 + j) P + p] = part p of row n's
// k group j, scaled by the row's s_n (P 2: hi and lo, pair2; P 3: hi, mid and
// lo, pair3, W exactly); then at byte N K 2 P the N inverse scales 1 / s_n.
// One workgroup a row: its largest |x|, then its groups.
template <int P>
__global__ void __launch_bounds__(256) pair_rows_kernel(const float* __restrict__ W, int N, int K, int64_t ldw,
                                                         bool transposed, u4* __restrict__ out) {
  static_assert(P == 2 || P == 3, "two or three parts");
  __shared__ float red[4];
  const int n = blockIdx.x, tid = threadIdx.x, KG = K / 8;
  auto at = [&](int k) { return transposed ? W[int64_t(k) * ldw + n] : W[int64_t(n) * ldw + k]; };
  float m = 0.f;
  for (int k = tid; k < K; k += 256) m = fmaxf(m, fabsf(at(k)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  const float s = pair_scale(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  for (int j = tid; j < KG; j += 256) {
    u4 pt[P];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = at(8 * j + 2 * e) * s, y = at(8 * j + 2 * e + 1) * s;
      unsigned h, md, lw;
      if constexpr (P == 2) {
        pair2(x, y, h, lw);
        pt[0][e] = h, pt[1][e] = lw;
      } else {
        pet_split::pair3(x, y, h, md, lw);
        pt[0][e] = h, pt[1][e] = md, pt[2][e] = lw;
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) out[(int64_t(n) * KG + j) * P + p] = pt[p];
  }
  if (tid == 0) reinterpret_cast<float*>(out + int64_t(N) * KG * P)[n] = 1.f / s;
}

// Rows of an activation X [M, K] (ld ldx) as fp16 pairs in pair_rows_kernel's
// layout (the M inverse scales after the pairs), one wave a row: lane j takes
// k groups j, j + 64, ..., held in registers from the row's largest |x| to
// its split (NGL groups a lane; NGL 0: any K, the row read twice, the second
// time from cache). Each lane writes 32 contiguous bytes a group.
template <int NGL>
__global__ void __launch_bounds__(256) pair_act_kernel(const float* __restrict__ X, int M, int K, int64_t ldx,
                                                        u4* __restrict__ out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63, KG = K / 8;
  if (row >= M) return;
  const float* x = X + int64_t(row) * ldx;
  constexpr int NV = NGL > 0 ? 2 * NGL : 2;
  float4 v[NV];
  float m = 0.f;
  auto amax = [](const float4& a) { return fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))); };
  if constexpr (NGL > 0) {
#pragma unroll
    for (int i = 0; i < NGL; ++i) {
      const int j = l + 64 * i;
      if (j < KG) {
        v[2 * i] = *reinterpret_cast<const float4*>(x + 8 * j);
        v[2 * i + 1] = *reinterpret_cast<const float4*>(x + 8 * j + 4);
        m = fmaxf(m, fmaxf(amax(v[2 * i]), amax(v[2 * i + 1])));
      }
    }
  } else {
    for (int j = l; j < KG; j += 64)
      m = fmaxf(m, fmaxf(amax(*reinterpret_cast<const float4*>(x + 8 * j)),
                         amax(*reinterpret_cast<const float4*>(x + 8 * j + 4))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  const float s = pair_scale(m);
  auto put = [&](int j, const float4& a, const float4& b) {
    u4 hi, lo;
    unsigned h, lw;
    pair2(a.x * s, a.y * s, h, lw), hi[0] = h, lo[0] = lw;
    pair2(a.z * s, a.w * s, h, lw), hi[1] = h, lo[1] = lw;
    pair2(b.x * s, b.y * s, h, lw), hi[2] = h, lo[2] = lw;
    pair2(b.z * s, b.w * s, h, lw), hi[3] = h, lo[3] = lw;
    u4* o = out + (int64_t(row) * KG + j) * 2;
    o[0] = hi, o[1] = lo;
  };
  if constexpr (NGL > 0) {
#pragma unroll
    for (int i = 0; i < NGL; ++i)
      if (l + 64 * i < KG) put(l + 64 * i, v[2 * i], v[2 * i + 1]);
  } else {
    for (int j = l; j < KG; j += 64)
      put(j, *reinterpret_cast<const float4*>(x + 8 * j), *reinterpret_cast<const float4*>(x + 8 * j + 4));
  }
  if (l == 0) reinterpret_cast<float*>(out + int64_t(M) * KG * 2)[row] = 1.f / s;
}

// The K loop's barrier: no memory fence, since any fence, even one on LDS
// alone, makes the compiler wait for every global-to-LDS load in flight (the
// prefetches too). The loop's own vmcnt wait before it covers the step's
// loads; an explicit lgkmcnt(0) wait (vmcnt and expcnt left at their maxima)
// makes every LDS read a wave issued in the step before complete before it
// passes, so no wave's global_load_lds can overwrite a stage another is still
// reading, whatever order the compiler gives the products; the empty asm
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}


// 16 bytes a lane from global memory into LDS, a wave's 64 lanes filling
// dst .. dst + 1 KB in lane order (dst wave-uniform). A device function: the
// builtin, called in a lambda of a kernel, stops the host side from emitting
// the kernel.
__device__ __forceinline__ void ring_load(const u4* src, u4* dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// s_waitcnt on the vector-memory counter alone (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14; expcnt 7 and lgkmcnt 15 wait for nothing).
template <int n>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// C = epi(A B^T) with both operands as fp16 pairs (pair_act_kernel's and
// pair_rows_kernel's layout): a row's K step of 32 is 8 u4, part p = 2 group +
// (0 hi, 1 lo). No vector arithmetic in the K loop: the steps go from global
// memory straight into an LDS ring of ST stages (global_load_lds_dwordx4, a
// wave's instruction filling 8 rows' steps, 1 KB), ST - 1 steps in flight, one
// barrier a step. Part p of row r sits in 16-byte slot p ^ f(r) of the row's
// 128 bytes, f(r) = bit 2 of r as bit 0 and bit 3 as bit 2: a 128-bit LDS
// read serves 32 lanes (16 rows, two k groups) a cycle over 128 banks, rows
// r, r + 4, r + 8, r + 12 share banks, and f gives their two groups' slots
// {x, x ^ 2} four disjoint pairs (measured: f = r & 7 2-way conflicts, 17% of
// cycles; f = (r >> 1) & 7 25%). The swizzle is applied on the global side
// (lane L of an instruction loads the part its slot L % 8 holds). The k order and the
// epilogue's unscaling are gemm_nt_pair_kernel's, so the two give the same bits.
// Tiles of WGM x WGN waves; K a multiple of 32.
// KBS > 0: A as block pairs (a staged epilogue's pout): A's scale is per (row,
// K block of 32 KBS), the inverse scales [K / (32 KBS)][M] after the pairs.
// Each block's products go to their own accumulators (cleared at the block's
// start), which are then added into the total times the rows'
// inverse scales for the block (staged in LDS after the ring at the start);
// B's column scales are undone at the end.
// PO: the output as block pairs (Epi::pout) from the staged epilogue.
template <int BM, int BN, int WGM, int WGN, int ST, int KBS = 0, bool PO = false>
__global__ void __launch_bounds__(64 * WGM * WGN)
__attribute__((amdgpu_waves_per_eu(BM == 128 && BN == 128 ? 4 : 1))) gemm_pp_kernel(int M, int N, int K, const u4* __restrict__ Ap,
                                                                  const u4* __restrict__ Bs, float* C, int64_t ldc,
                                                                  Epi epi, int WR) {
  constexpr int NW = WGM * WGN, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
  constexpr int SR = BM + BN, LPW = SR / 8 / NW;  // rows a stage; load instructions a wave a step
  static_assert(LPW * 8 * NW == SR && ST >= 2 && ST <= 6, "a stage's rows divide over the waves");
  extern __shared__ u4 ring[];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int wm = w / WGN, wn = w % WGN;
  // the XCD-contiguous tile order of gemm_nt_pair_kernel, one tile an item;
  // within an XCD's run, windows of WR row blocks, each swept column tile by
  // column tile with its row blocks fastest: the tiles in flight at once are
  // a few row blocks by a few column tiles, whose A rows and B strip both
  // stay in the XCD's L2 (row-block order instead streamed all of B, 4 MB at
  // N 2048, through each row block: 2.6 times the product's bytes)
  const int NT = (N + BN - 1) / BN, RB = (M + BM - 1) / BM, total = gridDim.x, L = blockIdx.x;
  const int q = total / 8, r = total % 8, x = L % 8;
  const int t = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + L / 8;
  const int wi = t / (WR * NT), wr = min(WR, RB - wi * WR), within = t - wi * WR * NT;
  const int m0 = (wi * WR + within % wr) * BM, n0 = (within / wr) * BN, KG = K / 8;

  // this lane's source for each of the wave's load instructions: stage row
  // R = 8 (w LPW + i) + l / 8 (A rows first, then B), part (l % 8) ^ (l / 8)
  const u4* src[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int R = 8 * (w * LPW + i) + (l >> 3), p = (l & 7) ^ (((R >> 2) & 1) | ((R >> 1) & 4));
    src[i] = R < BM ? Ap + int64_t(min(m0 + R, M - 1)) * KG * 2 + p
                    : Bs + int64_t(min(n0 + R - BM, N - 1)) * KG * 2 + p;
  }
  const int steps = K / 32;
  auto issue = [&](int s) {
    u4* dst = ring + (s % ST) * SR * 8 + w * LPW * 64;
#pragma unroll
    for (int i = 0; i < LPW; ++i)
      ring_load(src[i] + 8 * s, dst + 64 * i);
  };
  f4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
  // block pairs: the tile's rows' inverse scales of every K block into LDS
  // after the ring (the loads issued before the ring's first steps, the
  // stores after them)
  constexpr int SPT = KBS > 0 ? (32 * BM + 64 * NW - 1) / (64 * NW) : 1;  // scales a thread, at most 32 blocks
  float* scl = reinterpret_cast<float*>(ring + ST * SR * 8);
  const int nblk = KBS > 0 ? steps / KBS : 0;
  float sv[SPT];
  if constexpr (KBS > 0) {
    const float* inv_a = reinterpret_cast<const float*>(Ap + int64_t(M) * KG * 2);
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int ti = tid + 64 * NW * u, kb = ti / BM, rw = ti % BM;
      sv[u] = kb < nblk ? inv_a[int64_t(kb) * M + min(m0 + rw, M - 1)] : 0.f;
    }
  }
#pragma unroll
  for (int s = 0; s < ST - 1; ++s)
    if (s < steps) issue(s);
  if constexpr (KBS > 0) {
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int ti = tid + 64 * NW * u;
      if (ti < nblk * BM) scl[ti] = sv[u];
    }
  }
  const int fc = ((c >> 2) & 1) | ((c >> 1) & 4);  // f(row), row & 15 = c
  const int sw0 = (2 * g) ^ fc, sw1 = (2 * g + 1) ^ fc;
  // step s: its loads done (those after it may still fly), every wave's
  // reads of the stage it refills done, the refill issued, the products
  auto step = [&](int s) {
    const int after = min(ST - 2, steps - 1 - s);
    if (after >= ST - 2) wait_vm<(ST - 2) * LPW>();
    else if constexpr (ST >= 4) {
      if (after == 1) wait_vm<LPW>();
      else if (ST >= 5 && after == 2) wait_vm<2 * LPW>();
      else if (ST >= 6 && after == 3) wait_vm<3 * LPW>();
      else wait_vm<0>();
    } else {
      wait_vm<0>();
    }
    ring_barrier();
    if (s + ST - 1 < steps) issue(s + ST - 1);  // into the stage step s - 1 used
    const u4* st = ring + (s % ST) * SR * 8;
    u4 av[TM][2], bv[TN][2];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const u4* row = st + (wm * WM + 16 * a + c) * 8;
      av[a][0] = row[sw0], av[a][1] = row[sw1];
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const u4* row = st + (BM + wn * WN + 16 * b + c) * 8;
      bv[b][0] = row[sw0], bv[b][1] = row[sw1];
    }
    // mfma3's three products (hi lo, lo hi, hi hi), each over every tile
    // before the next: TM TN independent accumulators between two dependent
    // instructions, the same sums in the same order
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = pet_split::mfma_h(av[a][p == 0 ? 1 : 0], bv[b][p == 1 ? 1 : 0], acc[a][b]);
  };
  const float* inv_b = reinterpret_cast<const float*>(Bs + int64_t(N) * KG * 2);
  if constexpr (KBS == 0) {
    for (int s = 0; s < steps; ++s) step(s);
    const float* inv_a = reinterpret_cast<const float*>(Ap + int64_t(M) * KG * 2);
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float ib = inv_b[min(n0 + wn * WN + 16 * b + c, N - 1)];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          acc[a][b][rr] = acc[a][b][rr] * inv_a[min(m0 + wm * WM + 16 * a + 4 * g + rr, M - 1)] * ib;
    }
  } else {
    f4 tot[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) tot[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nblk; ++kb) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
      for (int ss = 0; ss < KBS; ++ss) step(kb * KBS + ss);
      // the block into the total, times its rows' inverse scales (rows 4g .. 4g + 3 of each tile)
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const float4 ia = *reinterpret_cast<const float4*>(scl + kb * BM + wm * WM + 16 * a + 4 * g);
        const float iar[4] = {ia.x, ia.y, ia.z, ia.w};
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) tot[a][b][rr] = fmaf(acc[a][b][rr], iar[rr], tot[a][b][rr]);
      }
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float ib = inv_b[min(n0 + wn * WN + 16 * b + c, N - 1)];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) acc[a][b][rr] = tot[a][b][rr] * ib;
    }
  }
  static_assert(ST * (BM + BN) * 128 >= BM * BN * 4, "the ring holds the result tile");
  if (staged_epilogue<BM, BN, WGM, WGN, 1, PO>(acc, reinterpret_cast<float*>(ring), m0, n0, M, N, C, ldc, epi)) return;
  if constexpr (!PO) epilogue<WM, WN>(acc, m0, n0, wm, wn, c, g, M, N, C, ldc, epi);  // (block pairs: the host makes sure of the staged one)
}

// epi_elem's arithmetic, in its order, for four consecutive output columns
// j .. j + 3 of row i (j a multiple of 4; a SwiGLU pair in one lane), with
// 16-byte accesses where vec (every pointer 16-byte aligned, every leading
// dimension and N multiples of 4), element by element otherwise.
template <bool vec, bool bwd>
__device__ __forceinline__ void epi_quad(float (&v)[4], int i, int j, int M, int N, float* C, int64_t ldc,
                                         const Epi& epi, const float4* bq = nullptr) {
  if (i >= M || j >= N) return;
  if constexpr (bwd) {
    const float* z = epi.cin + int64_t(i) * epi.ldcin;
    if constexpr (vec) {  // z, bias and C rows 16-byte aligned, N a multiple of 4
      if (epi.act == 3) {
        const float4 z4 = *reinterpret_cast<const float4*>(z + j);
        const float4 b4 = epi.bias ? *reinterpret_cast<const float4*>(epi.bias + j) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float xs[4] = {z4.x + b4.x, z4.y + b4.y, z4.z + b4.z, z4.w + b4.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sg = sig_fast(xs[e]);
          o[e] = v[e] * (sg * (1.0f + xs[e] * (1.0f - sg)));
        }
        *reinterpret_cast<float4*>(C + int64_t(i) * ldc + j) = make_float4(o[0], o[1], o[2], o[3]);
      } else {  // (value, gate) pairs 2 j .. 2 j + 7
        float zz[8];
        *reinterpret_cast<float4*>(zz) = *reinterpret_cast<const float4*>(z + 2 * j);
        *reinterpret_cast<float4*>(zz + 4) = *reinterpret_cast<const float4*>(z + 2 * j + 4);
        if (epi.bias) {
          const float4 b0 = *reinterpret_cast<const float4*>(epi.bias + 2 * j);
          const float4 b1 = *reinterpret_cast<const float4*>(epi.bias + 2 * j + 4);
          zz[0] += b0.x, zz[1] += b0.y, zz[2] += b0.z, zz[3] += b0.w;
          zz[4] += b1.x, zz[5] += b1.y, zz[6] += b1.z, zz[7] += b1.w;
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = zz[2 * e], sg = sig_fast(zz[2 * e + 1]);
          o[2 * e] = v[e] * sg;
          o[2 * e + 1] = v[e] * u * sg * (1.0f - sg);
        }
        float* cr = C + int64_t(i) * ldc + 2 * j;
        *reinterpret_cast<float4*>(cr) = make_float4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<float4*>(cr + 4) = make_float4(o[4], o[5], o[6], o[7]);
      }
      return;
    }
    if (epi.act == 3) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!vec && j + e >= N) break;
        const float x = z[j + e] + (epi.bias ? epi.bias[j + e] : 0.f), sg = sig_fast(x);
        o[e] = v[e] * (sg * (1.0f + x * (1.0f - sg)));
        if (!vec) C[int64_t(i) * ldc + j + e] = o[e];
      }
      if (vec) *reinterpret_cast<float4*>(C + int64_t(i) * ldc + j) = make_float4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (j + e >= N) break;
        const int jj = j + e;
        const float u = z[2 * jj] + (epi.bias ? epi.bias[2 * jj] : 0.f);
        const float sg = sig_fast(z[2 * jj + 1] + (epi.bias ? epi.bias[2 * jj + 1] : 0.f));
        *reinterpret_cast<float2*>(C + int64_t(i) * ldc + 2 * jj) = make_float2(v[e] * sg, v[e] * u * sg * (1.0f - sg));
      }
    }
    return;
  }
  const int ne = vec ? 4 : min(4, N - j);
  if (epi.row_scale) {
    const float rs = epi.row_scale[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= rs;
  }
  if (epi.bias) {
    if (vec) {
      const float4 b4 = bq ? *bq : *reinterpret_cast<const float4*>(epi.bias + j);
      v[0] += b4.x, v[1] += b4.y, v[2] += b4.z, v[3] += b4.w;
    } else {
      for (int e = 0; e < ne; ++e) v[e] += epi.bias[j + e];
    }
  }
  if (epi.cin) {
    const float* ci = epi.cin + int64_t(i) * epi.ldcin + j;
    if (vec) {
      const float4 c4 = *reinterpret_cast<const float4*>(ci);
      v[0] += epi.beta * c4.x, v[1] += epi.beta * c4.y, v[2] += epi.beta * c4.z, v[3] += epi.beta * c4.w;
    } else {
      for (int e = 0; e < ne; ++e) v[e] += epi.beta * ci[e];
    }
  }
  if (epi.pre) {
    float* pr = epi.pre + int64_t(i) * epi.ldpre + j;
    if (vec) {
      *reinterpret_cast<float4*>(pr) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < ne; ++e) pr[e] = v[e];
    }
  }
  float* ci = C + int64_t(i) * ldc;
  if (epi.act == 2) {  // N even: pairs (j, j + 1), (j + 2, j + 3)
    const float o0 = v[0] * sig_fast(v[1]), o1 = v[2] * sig_fast(v[3]);
    if (vec) {
      *reinterpret_cast<float2*>(ci + j / 2) = make_float2(o0, o1);
    } else {
      ci[j / 2] = o0;
      if (ne > 2) ci[j / 2 + 1] = o1;
    }
    return;
  }
  if (epi.act == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] * sig_fast(v[e]);
  }
  if (vec) {
    *reinterpret_cast<float4*>(ci + j) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    for (int e = 0; e < ne; ++e) ci[j + e] = v[e];
  }
}

// Small K (at most 128), weights in registers. A workgroup of four waves
// owns four groups of 16 TN output columns, one a wave, each holding its
// columns' weights as three fp16 parts in registers (loaded once, TN KB 12
// registers), and streams 16-row blocks of A: per block each thread takes one
// k group of 8 (a row's groups in KL consecutive lanes, KL the power of two at
// or above K / 8), the row's largest |x| comes from a shuffle over those
// lanes, and the rows are split into fp16 pairs once for the workgroup into a
// double-buffered LDS slice (rows padded to an odd number of 16-byte slots, so
// that the 16 rows a fragment read meets fall on distinct banks); the thread
// then loads its group of the next block into the registers it has just read.
// After one barrier each wave reads its operand fragments and runs the five
// part products per k group (a_hi and a_lo against w_hi and w_mid, and a_hi
// w_lo; the dropped a_lo w_lo is below 2^-33 of |a||w|), the column tiles'
// accumulations interleaved, with the weights as the instruction's first
// operand: lane (c, g) then holds output row c, columns 4 g .. 4 g + 3 of
// each 16-column tile, and the epilogue reads and writes 16 bytes a lane.
// XCD x (workgroup L on x = L mod 8) takes rows [x M / 8, (x + 1) M / 8) in S
// ranges per set of four column groups, so the sets re-read a range of A
// from their XCD's L2. A row's results depend on that row alone, and the
// products are summed in the order of the LDS-staged kernel this replaced:
// the same bits.
template <int KB, int TN, bool VEC, bool BWD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TN * KB <= 2 ? 4 : TN * KB <= 4 && !BWD ? 3 : 2)))
gemm_skt_kernel(int M, int N, const float* __restrict__ A, int64_t lda, const u4* __restrict__ Bp, float* C,
                int64_t ldc, Epi epi, int S) {
  // RB 16-row tiles a block (2, with twice the rows in flight, crashes the
  // ROCm 7.2 compiler's copy propagation at K = 128)
  constexpr int RB = 1;
  constexpr int KG = 4 * KB, CW = 16 * TN, RP = 2 * KG + 1, NW = 4, T = 64 * NW, R = 16 * RB;
  __shared__ u4 sa[2][R * RP];
  __shared__ float sinv[2][R];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int CG = (N + CW - 1) / CW, CS = (CG + NW - 1) / NW, x = blockIdx.x % 8, li = blockIdx.x / 8;
  if (li >= CS * S) return;  // (uniform over the workgroup)
  const int cs = li % CS, rs = li / CS, cg = cs * NW + w, n0 = cg * CW;
  const bool live = cg < CG;  // a wave past the last column group still splits rows for the others
  const int xr0 = int(int64_t(x) * M / 8), xr1 = int(int64_t(x + 1) * M / 8);
  const int nb = (xr1 - xr0 + R - 1) / R;
  const int b0 = int(int64_t(rs) * nb / S), b1 = int(int64_t(rs + 1) * nb / S);
  if (b0 >= b1) return;  // (uniform)
  u4 wh[TN][KB], wm[TN][KB], wl[TN][KB];
  float ib[TN][4];
  {
    const float* inv_b = reinterpret_cast<const float*>(Bp + int64_t(N) * KG * 3);
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const u4* br = Bp + int64_t(min(n0 + 16 * b + c, N - 1)) * (3 * KG);
#pragma unroll
      for (int kk = 0; kk < KB; ++kk) {
        wh[b][kk] = br[(4 * kk + g) * 3];
        wm[b][kk] = br[(4 * kk + g) * 3 + 1];
        wl[b][kk] = br[(4 * kk + g) * 3 + 2];
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) ib[b][rr] = inv_b[min(n0 + 16 * b + 4 * g + rr, N - 1)];
    }
  }
  constexpr bool HB = VEC && !BWD;  // a forward epilogue with 16-byte accesses: the bias held
  float4 bq[HB ? TN : 1];
  if constexpr (HB) {
#pragma unroll
    for (int b = 0; b < TN; ++b)
      bq[b] = epi.bias && live ? *reinterpret_cast<const float4*>(epi.bias + min(n0 + 16 * b + 4 * g, N - 4))
                               : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // a thread's k groups of a block: item e = tid + T q, row e / KL, group
  // e % KL (KL the power of two at or above KG: a row's groups are KL
  // consecutive lanes of one wave, those at KG and above idle); loaded one
  // block ahead, into the registers the split has just read
  constexpr int KL = KG <= 4 ? 4 : KG <= 8 ? 8 : 16, ITEMS = R * KL, NI = (ITEMS + T - 1) / T;
  static_assert(ITEMS % T == 0 || ITEMS < T, "whole passes");
  float4 v0[NI], v1[NI];
  auto load_a = [&](int blk) {
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int e = tid + T * q;
      if (e < ITEMS && e % KL < KG) {
        const float* p = A + int64_t(min(xr0 + R * blk + e / KL, xr1 - 1)) * lda + 8 * (e % KL);
        v0[q] = *reinterpret_cast<const float4*>(p);
        v1[q] = *reinterpret_cast<const float4*>(p + 4);
      } else {
        v0[q] = v1[q] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  load_a(b0);
  for (int blk = b0; blk < b1; ++blk) {
    const int buf = (blk - b0) & 1;
#pragma unroll
    for (int q = 0; q < NI; ++q) {
      const int e = tid + T * q, ir = e / KL, ij = e % KL;
      float m = fmaxf(fmaxf(fmaxf(fabsf(v0[q].x), fabsf(v0[q].y)), fmaxf(fabsf(v0[q].z), fabsf(v0[q].w))),
                      fmaxf(fmaxf(fabsf(v1[q].x), fabsf(v1[q].y)), fmaxf(fabsf(v1[q].z), fabsf(v1[q].w))));
#pragma unroll
      for (int o = 1; o < KL; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));  // the row's KL consecutive lanes
      const float sc = pair_scale(m);
      unsigned h[4], lo[4];
      pair2(v0[q].x * sc, v0[q].y * sc, h[0], lo[0]);
      pair2(v0[q].z * sc, v0[q].w * sc, h[1], lo[1]);
      pair2(v1[q].x * sc, v1[q].y * sc, h[2], lo[2]);
      pair2(v1[q].z * sc, v1[q].w * sc, h[3], lo[3]);
      if (e < ITEMS && ij < KG) {
        sa[buf][ir * RP + 2 * ij] = u4{h[0], h[1], h[2], h[3]};
        sa[buf][ir * RP + 2 * ij + 1] = u4{lo[0], lo[1], lo[2], lo[3]};
        if (ij == 0) sinv[buf][ir] = 1.f / sc;
      }
    }
    load_a(min(blk + 1, b1 - 1));  // (the last block's rows again at the end: in bounds, unused)
    __syncthreads();  // the block's pairs are in LDS; (double buffer) no wave still reads the slice two blocks back
    if (live) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        u4 ah[KB], al[KB];
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
          ah[kk] = sa[buf][(16 * r + c) * RP + 2 * (4 * kk + g)];
          al[kk] = sa[buf][(16 * r + c) * RP + 2 * (4 * kk + g) + 1];
        }
        const float isc = sinv[buf][16 * r + c];
        const int i = xr0 + R * blk + 16 * r + c;
        // the tiles' chains interleaved (each tile's products in the same
        // order, small ones first), so TN independent accumulations are in
        // flight
        f4 acc[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[b] = pet_split::mfma_h(wm[b][kk], al[kk], acc[b]);
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[b] = pet_split::mfma_h(wl[b][kk], ah[kk], acc[b]);
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[b] = pet_split::mfma_h(wh[b][kk], al[kk], acc[b]);
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[b] = pet_split::mfma_h(wm[b][kk], ah[kk], acc[b]);
#pragma unroll
          for (int b = 0; b < TN; ++b) acc[b] = pet_split::mfma_h(wh[b][kk], ah[kk], acc[b]);
        }
#pragma unroll
        for (int b = 0; b < TN; ++b) {
          float o[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) o[rr] = acc[b][rr] * isc * ib[b][rr];
          if (i < xr1)
            epi_quad<VEC, BWD>(o, i, n0 + 16 * b + 4 * g, M, N, C, ldc, epi, HB ? &bq[HB ? b : 0] : nullptr);
          // (one tile's epilogue at a time: its loads are not hoisted above
          // the last tile's stores, which would hold every tile's operands)
          asm volatile("" ::: "memory");
        }
      }
    }
  }
}

}  // namespace pet_gemm

using namespace pet_gemm;

// Which split a K takes: fp16 pairs from K = 256 (three matrix instructions a
// product where the bf16 form takes six, and a first pass over A's rows for
// their scales, which pays once the K loop is long enough: measured 131072 x
// 1536 x 512 908-923 against 1220 us, 122688 x 768 x 256 289 against 345 us,
// but 26670 x 1024 x 128 78 against 70 us), three bf16 parts below. The
// weights' split and the product both follow it, so a split copy matches the
// kernel that reads it.
static bool pair_form(int K) { return K >= 256; }

// The tile shape for a problem: wide outputs take 128 x 128; narrow ones
// (N <= 64) or too few tiles to fill 256 CUs take smaller tiles.
int pet_gemm_nt_fused(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta, float* pre,
                int64_t ldpre, int act, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (K == 0) return PET_ATTN_EINVAL;
  if (K % 16 || lda % 4 || ldb % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(B) & 15))
    return PET_ATTN_EALIGN;
  if (act == 2 && N % 2) return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  auto tiles = [&](int bm, int bn) { return int64_t((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  const bool k32 = K % 32 == 0;
  auto go = [&](auto kern, int bm, int bn) {  // a 1-D grid: every tile, no extent limit below 2^31 tiles
    hipLaunchKernelGGL(kern, dim3(unsigned(tiles(bm, bn))), dim3(256), 0, st, M, N, K, A, lda, B, ldb, C, ldc, e);
  };
  if (tiles(64, 32) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  if (N > 64 && tiles(128, 128) >= 512)
    k32 ? go(gemm_nt_kernel<128, 128, 32>, 128, 128) : go(gemm_nt_kernel<128, 128, 16>, 128, 128);
  else if (N > 32 && tiles(128, 64) >= 512)
    k32 ? go(gemm_nt_kernel<128, 64, 32>, 128, 64) : go(gemm_nt_kernel<128, 64, 16>, 128, 64);
  else
    k32 ? go(gemm_nt_kernel<64, 32, 32>, 64, 32) : go(gemm_nt_kernel<64, 32, 16>, 64, 32);
  tally(0, M, N, K);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// The epilogue arguments of the public entry points: C's and cin's widths
// per act (act 4 writes and reads 2N columns), cin required by the backward
// codes 3 and 4, which take no row scale and no pre.
static bool epi_args_ok(int N, const float* C, int64_t ldc, const float* row_scale, const float* cin, int64_t ldcin,
                        const float* pre, int64_t ldpre, int act) {
  if (act < 0 || act > 4 || !C) return false;
  if (act >= 3) {
    const int64_t w = act == 4 ? 2 * int64_t(N) : N;
    // act 4 stores (value, gate) adjoint pairs as 8-byte words
    const bool pairs_ok = act == 3 || ((reinterpret_cast<uintptr_t>(C) & 7) == 0 && ldc % 2 == 0);
    return cin && ldcin >= w && ldc >= w && !row_scale && !pre && pairs_ok;
  }
  return ldc >= (act == 2 ? N / 2 : N) && (!cin || ldcin >= N) && (!pre || ldpre >= N);
}

extern "C" int pet_linear_fused(int M, int N, int K, const float* A, int64_t lda, const float* W, int64_t ldw,
                                float* C, int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!A || !W || !C || lda < K || ldw < K || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin,
                                                                                    pre, ldpre, act)))
    return PET_ATTN_EINVAL;
  return pet_gemm_nt_fused(M, N, K, A, lda, W, ldw, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre, act,
                           reinterpret_cast<hipStream_t>(stream));
}

int pet_gemm_nt_pp(int M, int N, int K, const void* Ap, const void* Bs, float* C, int64_t ldc, const Epi& e,
                   hipStream_t st, bool tile128 = false);
int pet_gemm_pair_rows(const float* X, int M, int K, int64_t ldx, void* out, hipStream_t st);

// The pairs-by-pairs path's threshold: from N = 512 the products' gain
// outweighs splitting A (C5 energy+forces on MI355X, same bits: N >= 1024
// 176.4 ms, N >= 512 171.4, N >= 256 171.4, never 191; plain products, same
// process: 131072 x 1536 x 512 1060 against 95 + 800 us, 498338 x 2048 x 512
// 4634 against 342 + 3443; with a kept pre-activation 5760 against 4244).
constexpr int kPairsMinN = 512;

// The split-product GEMM with the epilogue e (block pairs out where e.pout:
// then 128 x 128 tiles, so that an output row's K blocks are 128 columns of
// the product wide).
int split_impl(int M, int N, int K, const float* A, int64_t lda, const void* Bs, float* C, int64_t ldc, Epi e,
               hipStream_t st, void* scratch, size_t scratch_bytes) {
  if (M < 0 || N < 0 || K < 0) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (K == 0) return PET_ATTN_EINVAL;
  if (int64_t((M + 63) / 64) * ((N + 63) / 64) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;  // 1-D grid of tiles
  if (K % 32 || lda % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(Bs) & 15))
    return PET_ATTN_EALIGN;
  if (e.act == 2 && N % 2) return PET_ATTN_EINVAL;
  const int64_t ldcin = e.ldcin, ldpre = e.ldpre;
  const bool t128 = e.pout != nullptr;
  // A's rows split into the scratch a chunk at a time (as many rows as it
  // holds, a multiple of 128), each chunk's product from the pairs
  const int64_t chunk = scratch ? int64_t(scratch_bytes / (size_t(K) * 4 + 4)) / 128 * 128 : 0;
  const bool pp = pair_form(K) && N >= kPairsMinN && chunk >= 128 && (reinterpret_cast<uintptr_t>(scratch) & 15) == 0;
  if (t128 && !pp) return PET_ATTN_EINVAL;  // block pairs out: the pairs-by-pairs kernel only
  if (pp) {
    for (int64_t r0 = 0; r0 < M; r0 += chunk) {
      const int m = int(std::min<int64_t>(chunk, M - r0));
      Epi ec = e;
      if (ec.row_scale) ec.row_scale += r0;
      if (ec.cin) ec.cin += r0 * ldcin;
      if (ec.pre) ec.pre += r0 * ldpre;
      if (ec.pout) ec.pout += r0 * ec.kgo * 2, ec.pinv += r0;
      int rc = pet_gemm_pair_rows(A + r0 * lda, m, K, lda, scratch, st);
      if (rc == PET_ATTN_OK) rc = pet_gemm_nt_pp(m, N, K, scratch, Bs, C ? C + r0 * ldc : C, ldc, ec, st, t128);
      if (rc != PET_ATTN_OK) return rc;
    }
    return PET_ATTN_OK;
  }
  auto go = [&](auto kern, int bm, int bn, int threads, bool pair) {  // a 1-D grid of every work item
    const int64_t rb = (M + bm - 1) / bm, nt = (N + bn - 1) / bn;
    // column tiles per item (pair kernel): about 2048 items, four rounds of
    // two workgroups a CU (the rows' scales are found once an item; measured
    // against 1024, 1536 and 3072 items: 131072 x 1536 x 512 842 against
    // 883-850 us, 131072 x 512 x 2048 1062 against 1203-1055 us)
    const int64_t c0 = pair ? std::max<int64_t>(1, std::min<int64_t>(nt, rb * nt / 2048)) : 1;
    const int64_t ng = (nt + c0 - 1) / c0, cpw = (nt + ng - 1) / ng;
    hipLaunchKernelGGL(kern, dim3(unsigned(rb * ((nt + cpw - 1) / cpw))), dim3(threads), 0, st, M, N, K, A, lda,
                       static_cast<const u4*>(Bs), C, ldc, e, static_cast<const float*>(nullptr), int64_t(0),
                       int(cpw));
    tally(pair ? 2 : 1, M, N, K);
  };
  // measured on MI355X: 128 x 128 tiles of 8 waves where there are many
  // (131072 x 1536 x 512: 1200-1213 us against 1394-1418 for 128 x 64 and
  // 1535 for 64 x 64; 256 x 128 and 128 x 256 tiles of 16 waves were no
  // faster), 64 x 64 otherwise (27318 x 128 x 128: 16.1 against 18.4 us); one
  // LDS buffer beat two in every shape
  const int64_t tiles128 = int64_t((M + 127) / 128) * ((N + 63) / 64);
  if (pair_form(K)) {
    if (t128 || (N >= 128 && tiles128 >= 2048))
      go(gemm_nt_pair_kernel<128, 128, 2, 4>, 128, 128, 512, true);
    else if (tiles128 >= 2048)
      go(gemm_nt_pair_kernel<128, 64>, 128, 64, 256, true);
    else
      go(gemm_nt_pair_kernel<64, 64>, 64, 64, 256, true);
  } else {
    if (t128 || (N >= 128 && tiles128 >= 2048))
      go(gemm_nt_split_kernel<128, 128, 2, 4>, 128, 128, 512, false);
    else if (tiles128 >= 2048)
      go(gemm_nt_split_kernel<128, 64>, 128, 64, 256, false);
    else
      go(gemm_nt_split_kernel<64, 64>, 64, 64, 256, false);
  }
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

int pet_gemm_nt_split(int M, int N, int K, const float* A, int64_t lda, const void* Bs, float* C, int64_t ldc,
                      const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                      float* pre, int64_t ldpre, int act, hipStream_t st, void* scratch, size_t scratch_bytes) {
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  return split_impl(M, N, K, A, lda, Bs, C, ldc, e, st, scratch, scratch_bytes);
}

// The output columns of a product of N columns under activation act.
static int out_cols(int N, int act) { return act == 2 ? N / 2 : act == 4 ? 2 * N : N; }

// Block pairs out: the split-product GEMM's output epi(A B^T) as fp16 pairs
// scaled per (row, 128-column tile of the product) into pout -- M rows of
// out_cols(N, act) / 8 k groups (pair_act_kernel's layout), then the inverse
// scales [out_cols(N, act) / kb][M] -- for a product that reads them as its A
// (pet_gemm_nt_pp_blocks with that kb, returned in *kb: 64 for SwiGLU, 256
// for its backward, 128 otherwise). N a multiple of 128, the output's columns
// of 32, every epilogue operand 16-byte aligned with leading dimensions of 4.
int pet_gemm_nt_split_pairs(int M, int N, int K, const float* A, int64_t lda, const void* Bs, void* pout,
                            const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                            float* pre, int64_t ldpre, int act, hipStream_t st, void* scratch, size_t scratch_bytes,
                            int* kb) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const int no = out_cols(N, act);
  if (!pout || !a16(pout) || N % 128 || no % 32 || (bias && !a16(bias)) || (cin && (!a16(cin) || ldcin % 4)) ||
      (pre && (!a16(pre) || ldpre % 4)))
    return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  e.pout = static_cast<u4*>(pout), e.kgo = no / 8, e.ldinv = M;
  e.pinv = reinterpret_cast<float*>(e.pout + int64_t(M) * e.kgo * 2);
  if (kb) *kb = out_cols(128, act);
  return split_impl(M, N, K, A, lda, Bs, nullptr, 0, e, st, scratch, scratch_bytes);
}

// The same product from fp32 B [N, K] (ld ldb), split as it is staged: for
// callers with no room to keep a split copy of the weights (the op-level
// attention()'s output linear). K a multiple of 32; A and B 16-byte aligned
// rows.
int pet_gemm_nt_split_f32b(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                           int64_t ldc, const float* bias, const float* cin, int64_t ldcin, float beta, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (K == 0) return PET_ATTN_EINVAL;
  if (int64_t((M + 63) / 64) * ((N + 63) / 64) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  if (K % 32 || lda % 4 || ldb % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(B) & 15))
    return PET_ATTN_EALIGN;
  Epi e;
  e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta;
  auto go = [&](auto kern, int bm, int bn, int threads) {
    const int64_t tiles = int64_t((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    hipLaunchKernelGGL(kern, dim3(unsigned(tiles)), dim3(threads), 0, st, M, N, K, A, lda, nullptr, C, ldc, e, B,
                       ldb, 1);
    tally(1, M, N, K);
  };
  const int64_t t128 = int64_t((M + 127) / 128) * ((N + 63) / 64);
  if (N >= 128 && t128 >= 2048)
    go(gemm_nt_split_kernel<128, 128, 2, 4, true>, 128, 128, 512);
  else if (t128 >= 2048)
    go(gemm_nt_split_kernel<128, 64, 2, 2, true>, 128, 64, 256);
  else
    go(gemm_nt_split_kernel<64, 64, 2, 2, true>, 64, 64, 256);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// B [N, K] as split rows, from W = B (transposed false: W [N, K]) or W = B^T
// (transposed true: W [K, N]); K a multiple of 32, out 16-byte aligned.
int pet_gemm_split_weights(const float* W, int N, int K, int64_t ldw, bool transposed, void* out, hipStream_t st) {
  if (N < 0 || K < 0 || K % 32 || (reinterpret_cast<uintptr_t>(out) & 15)) return PET_ATTN_EINVAL;
  const int64_t n = int64_t(N) * (K / 8);
  if (n == 0) return PET_ATTN_OK;
  if (pair_form(K))
    hipLaunchKernelGGL(pair_rows_kernel<2>, dim3(unsigned(N)), dim3(256), 0, st, W, N, K, ldw, transposed,
                       static_cast<u4*>(out));
  else if (transposed)
    hipLaunchKernelGGL(split_rows_t_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, W, N, K, ldw,
                       static_cast<u4*>(out));
  else
    hipLaunchKernelGGL(split_rows_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, W, N, K, ldw,
                       static_cast<u4*>(out));
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

extern "C" int pet_linear_split_weights(const float* W, int N, int K, int64_t ldw, void* out, void* stream) {
  if (N < 0 || K < 0 || K % 32 || ldw < K || ((N > 0 && K > 0) && (!W || !out))) return PET_ATTN_EINVAL;
  if (reinterpret_cast<uintptr_t>(out) & 15) return PET_ATTN_EALIGN;
  const int64_t n = int64_t(N) * (K / 8);
  if (n == 0) return PET_ATTN_OK;
  return pet_gemm_split_weights(W, N, K, ldw, false, out, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_linear_split_weights_transposed(const float* W, int N, int K, int64_t ldw, void* out,
                                                   void* stream) {
  if (N < 0 || K < 0 || K % 32 || ldw < N || ((N > 0 && K > 0) && (!W || !out))) return PET_ATTN_EINVAL;
  if (reinterpret_cast<uintptr_t>(out) & 15) return PET_ATTN_EALIGN;
  return pet_gemm_split_weights(W, N, K, ldw, true, out, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_linear_fused_split(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit, float* C,
                                      int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                      int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!A || !Wsplit || !C || lda < K || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin, pre,
                                                                              ldpre, act)))
    return PET_ATTN_EINVAL;
  return pet_gemm_nt_split(M, N, K, A, lda, Wsplit, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre, act,
                           reinterpret_cast<hipStream_t>(stream), nullptr, 0);
}

extern "C" int pet_linear_fused_split_ws(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit,
                                         float* C, int64_t ldc, const float* row_scale, const float* bias,
                                         const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre,
                                         int act, void* scratch, size_t scratch_bytes, void* stream) {
  if ((M > 0 && N > 0) && (!A || !Wsplit || !C || lda < K || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin, pre,
                                                                              ldpre, act)))
    return PET_ATTN_EINVAL;
  if (scratch_bytes && !scratch) return PET_ATTN_EINVAL;
  return pet_gemm_nt_split(M, N, K, A, lda, Wsplit, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre, act,
                           reinterpret_cast<hipStream_t>(stream), scratch, scratch_bytes);
}

// fp16-pair rows of an activation X [M, K] into out (M K 4 + M 4 bytes,
// 16-byte aligned): the A operand of pet_gemm_nt_pp. Pair-form K only.
int pet_gemm_pair_rows(const float* X, int M, int K, int64_t ldx, void* out, hipStream_t st) {
  if (M < 0 || K < 0 || !pair_form(K) || K % 32 || ldx % 4 || (reinterpret_cast<uintptr_t>(X) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 15))
    return PET_ATTN_EINVAL;
  if (M == 0) return PET_ATTN_OK;
  const dim3 grid(unsigned((M + 3) / 4));
  u4* o = static_cast<u4*>(out);
  if (K <= 512)
    hipLaunchKernelGGL(pair_act_kernel<1>, grid, dim3(256), 0, st, X, M, K, ldx, o);
  else if (K <= 1024)
    hipLaunchKernelGGL(pair_act_kernel<2>, grid, dim3(256), 0, st, X, M, K, ldx, o);
  else if (K <= 2048)
    hipLaunchKernelGGL(pair_act_kernel<4>, grid, dim3(256), 0, st, X, M, K, ldx, o);
  else
    hipLaunchKernelGGL(pair_act_kernel<0>, grid, dim3(256), 0, st, X, M, K, ldx, o);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// The pairs-by-pairs kernel's shapes: tile, waves, LDS stages.
struct PPShape {
  void (*kern)(int, int, int, const u4*, const u4*, float*, int64_t, Epi, int);
  int bm, bn, threads, stages;
  size_t lds() const { return size_t(stages) * (bm + bn) * 128; }
};
// measured on MI355X (131072 x 1536 x 512, plain epilogue): 128 x 128 tiles
// of 8 waves with two stages (two workgroups a CU) 752-813 us; four stages (one
// workgroup) 1128; three 991; 256 x 128 tiles, three stages 827-874; 128 x
// 128 of 4 waves 1300; the operand reads of the next step issued before this
// step's products (a second register set, three or four stages) 695-1018
const PPShape kPP[] = {
    {gemm_pp_kernel<128, 128, 2, 4, 2>, 128, 128, 512, 2},  // many tiles, N >= 128
    {gemm_pp_kernel<128, 64, 2, 2, 4>, 128, 64, 256, 4},    // fewer tiles, N >= 64
    {gemm_pp_kernel<64, 64, 2, 2, 4>, 64, 64, 256, 4},      // the rest
};
// the first shape with block pairs out (Epi::pout)
const PPShape kPPOut = {gemm_pp_kernel<128, 128, 2, 4, 2, 0, true>, 128, 128, 512, 2};

// C = epi(A B^T) from the pairs of A (pet_gemm_pair_rows) and of B
// (pet_gemm_split_weights), K of the pair form.
int pet_gemm_nt_pp(int M, int N, int K, const void* Ap, const void* Bs, float* C, int64_t ldc, const Epi& e,
                   hipStream_t st, bool tile128) {
  if (M < 0 || N < 0 || !pair_form(K) || K % 32) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if ((reinterpret_cast<uintptr_t>(Ap) & 15) || (reinterpret_cast<uintptr_t>(Bs) & 15)) return PET_ATTN_EALIGN;
  if (int64_t((M + 63) / 64) * ((N + 63) / 64) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  // each shape's dynamic LDS above the 64 KB default, set once a device (the
  // attribute is the current device's) for every shape
  static std::mutex mu;
  static signed char set_on[64] = {};  // 0 not yet, 1 set, -1 failed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PET_ATTN_ELAUNCH;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (set_on[dev] == 0) {
      set_on[dev] = 1;
      for (const PPShape& k : kPP)
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(k.kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                int(k.lds())) != hipSuccess)
          set_on[dev] = -1;
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(kPPOut.kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              int(kPPOut.lds())) != hipSuccess)
        set_on[dev] = -1;
    }
    if (set_on[dev] < 0) return PET_ATTN_ELAUNCH;
  }
  const int64_t t128 = int64_t((M + 127) / 128) * ((N + 127) / 128);
  const PPShape& k = e.pout ? kPPOut : kPP[tile128 || (N >= 128 && t128 >= 1024) ? 0 : N >= 64 ? 1 : 2];
  const int64_t tiles = int64_t((M + k.bm - 1) / k.bm) * ((N + k.bn - 1) / k.bn);
  // windows of 8 row blocks (498338 x 2048 x 512 on MI355X: L2-miss reads
  // 4.55 -> 2.71 GiB a product, 3587 -> 3428 us; 16 the same time, 2 and 4
  // between)
  constexpr int wr = 8;
  hipLaunchKernelGGL(k.kern, dim3(unsigned(tiles)), dim3(k.threads), k.lds(), st, M, N, K,
                     static_cast<const u4*>(Ap), static_cast<const u4*>(Bs), C, ldc, e, wr);
  tally(2, M, N, K);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// Block pairs out (as pet_gemm_nt_split_pairs) from A already as pair rows
// (pet_gemm_pair_rows' layout, K of the pair form): the pairs-by-pairs kernel
// alone, every row at once.
int pet_gemm_nt_pp_to_blocks(int M, int N, int K, const void* Ap, const void* Bs, void* pout, const float* bias,
                             const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre, int act,
                             hipStream_t st, int* kb) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const int no = out_cols(N, act);
  if (!pout || !a16(pout) || N % 128 || no % 32 || (bias && !a16(bias)) || (cin && (!a16(cin) || ldcin % 4)) ||
      (pre && (!a16(pre) || ldpre % 4)) || act < 0 || act > 4 || (act == 2 && N % 2))
    return PET_ATTN_EINVAL;
  Epi e;
  e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre, e.act = act;
  e.pout = static_cast<u4*>(pout), e.kgo = no / 8, e.ldinv = M;
  e.pinv = reinterpret_cast<float*>(e.pout + int64_t(M) * e.kgo * 2);
  if (kb) *kb = out_cols(128, act);
  return pet_gemm_nt_pp(M, N, K, Ap, Bs, nullptr, 0, e, st, true);
}

// The block-pairs product's kernels: kPP's shapes, by K block of 32, 64, 128
// or 256 (KBS 1, 2, 4, 8 steps); each takes at most 32 blocks' scales in LDS
// after its ring.
using PPKern = void (*)(int, int, int, const u4*, const u4*, float*, int64_t, Epi, int);
constexpr int kMaxBlocks = 32;
PPKern pp_blocks_kernel(int shape, int kbs) {
  switch (shape * 16 + kbs) {
    case 1: return gemm_pp_kernel<128, 128, 2, 4, 2, 1>;
    case 2: return gemm_pp_kernel<128, 128, 2, 4, 2, 2>;
    case 4: return gemm_pp_kernel<128, 128, 2, 4, 2, 4>;
    case 8: return gemm_pp_kernel<128, 128, 2, 4, 2, 8>;
    case 17: return gemm_pp_kernel<128, 64, 2, 2, 4, 1>;
    case 18: return gemm_pp_kernel<128, 64, 2, 2, 4, 2>;
    case 20: return gemm_pp_kernel<128, 64, 2, 2, 4, 4>;
    case 24: return gemm_pp_kernel<128, 64, 2, 2, 4, 8>;
    case 33: return gemm_pp_kernel<64, 64, 2, 2, 4, 1>;
    case 34: return gemm_pp_kernel<64, 64, 2, 2, 4, 2>;
    case 36: return gemm_pp_kernel<64, 64, 2, 2, 4, 4>;
    case 40: return gemm_pp_kernel<64, 64, 2, 2, 4, 8>;
    default: return nullptr;
  }
}

// C = epi(A B^T) with A as block pairs (pet_gemm_nt_split_pairs' pout: M
// rows of pairs, then the inverse scales [K / kb][M]) and B's pair rows; kb 32,
// 64, 128 or 256, dividing K, at most 32 blocks.
int pet_gemm_nt_pp_blocks(int M, int N, int K, const void* Ap, int kb, const void* Bs, float* C, int64_t ldc,
                          const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                          float* pre, int64_t ldpre, int act, hipStream_t st) {
  if (M < 0 || N < 0 || K <= 0 || K % 32 || !(kb == 32 || kb == 64 || kb == 128 || kb == 256) || K % kb ||
      K / kb > kMaxBlocks || (act == 2 && N % 2))
    return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if ((reinterpret_cast<uintptr_t>(Ap) & 15) || (reinterpret_cast<uintptr_t>(Bs) & 15)) return PET_ATTN_EALIGN;
  if (int64_t((M + 63) / 64) * ((N + 63) / 64) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  static std::mutex mu;
  static signed char set_on[64] = {};  // 0 not yet, 1 set, -1 failed
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return PET_ATTN_ELAUNCH;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (set_on[dev] == 0) {
      set_on[dev] = 1;
      for (int sh = 0; sh < 3; ++sh)
        for (int kbs : {1, 2, 4, 8})
          if (hipFuncSetAttribute(reinterpret_cast<const void*>(pp_blocks_kernel(sh, kbs)),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  int(kPP[sh].lds() + size_t(kMaxBlocks) * kPP[sh].bm * 4)) != hipSuccess)
            set_on[dev] = -1;
    }
    if (set_on[dev] < 0) return PET_ATTN_ELAUNCH;
  }
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  const int64_t t128 = int64_t((M + 127) / 128) * ((N + 127) / 128);
  const int sh = N >= 128 && t128 >= 1024 ? 0 : N >= 64 ? 1 : 2;
  const PPShape& k = kPP[sh];
  const int64_t tiles = int64_t((M + k.bm - 1) / k.bm) * ((N + k.bn - 1) / k.bn);
  const size_t lds = k.lds() + size_t(K / kb) * k.bm * 4;
  hipLaunchKernelGGL(pp_blocks_kernel(sh, kb / 32), dim3(unsigned(tiles)), dim3(k.threads), lds, st, M, N, K,
                     static_cast<const u4*>(Ap), static_cast<const u4*>(Bs), C, ldc, e, 8);
  tally(2, M, N, K);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// B's rows as three fp16 parts (hi, mid, lo: W exactly) at any K (a multiple
// of 32), for the short-K kernel: N K 6 + N 4 bytes.
int pet_gemm_pair_weights(const float* W, int N, int K, int64_t ldw, bool transposed, void* out, hipStream_t st) {
  if (N < 0 || K < 0 || K % 32 || (reinterpret_cast<uintptr_t>(out) & 15)) return PET_ATTN_EINVAL;
  if (N == 0 || K == 0) return PET_ATTN_OK;
  hipLaunchKernelGGL(pair_rows_kernel<3>, dim3(unsigned(N)), dim3(256), 0, st, W, N, K, ldw, transposed,
                     static_cast<u4*>(out));
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// C = epi(A B^T) for K at most 128 (a multiple of 32), B as rows of three
// fp16 parts (pet_gemm_pair_weights): gemm_skt_kernel.
int pet_gemm_nt_sk(int M, int N, int K, const float* A, int64_t lda, const void* Bp, float* C, int64_t ldc,
                   const Epi& e, hipStream_t st) {
  if (M < 0 || N < 0 || K < 32 || K > 128 || K % 32) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (lda % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(Bp) & 15))
    return PET_ATTN_EALIGN;
  // 32 columns a wave (64 at K <= 64, where the weights take half the
  // registers); about 64 workgroups an XCD (two a CU), the XCD's rows split
  // into S ranges per set of four column groups. Measured on MI355X at
  // 27318 rows (K 128, N 1024: 58 us against 78 for a 64 x 64-tile kernel
  // staging the weights through LDS; 32 and 128 workgroups an XCD slower).
  const int KB = K / 32, TN = KB <= 2 ? 4 : 2, CW = 16 * TN;
  const int64_t CG = (N + CW - 1) / CW, CS = (CG + 3) / 4;
  const int64_t rows_x = (M + 7) / 8, nbx = (rows_x + 15) / 16;
  const int64_t S = std::max<int64_t>(1, std::min<int64_t>(std::max<int64_t>(1, 64 / CS), nbx));
  const int64_t wgx = CS * S;
  if (wgx * 8 >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = N % 4 == 0 && a16(C) && ldc % 4 == 0 && (!e.bias || a16(e.bias)) &&
                   (!e.cin || (a16(e.cin) && e.ldcin % 4 == 0)) && (!e.pre || (a16(e.pre) && e.ldpre % 4 == 0));
  const u4* B = static_cast<const u4*>(Bp);
  const dim3 grid{unsigned(wgx * 8)}, block{256};
#define PET_SKT_LAUNCH(kb, tn, v, bw) \
  hipLaunchKernelGGL((gemm_skt_kernel<kb, tn, v, bw>), grid, block, 0, st, M, N, A, lda, B, C, ldc, e, int(S))
#define PET_SKT_GO(kb, tn)                    \
  if (e.act >= 3 && vec)                      \
    PET_SKT_LAUNCH(kb, tn, true, true);       \
  else if (e.act >= 3)                        \
    PET_SKT_LAUNCH(kb, tn, false, true);      \
  else if (vec)                               \
    PET_SKT_LAUNCH(kb, tn, true, false);      \
  else                                        \
    PET_SKT_LAUNCH(kb, tn, false, false)
  switch (KB) {
    case 1: PET_SKT_GO(1, 4); break;
    case 2: PET_SKT_GO(2, 4); break;
    case 3: PET_SKT_GO(3, 2); break;
    default: PET_SKT_GO(4, 2); break;
  }
#undef PET_SKT_GO
#undef PET_SKT_LAUNCH
  tally(3, M, N, K);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

extern "C" int pet_linear_pair_weights(const float* W, int N, int K, int64_t ldw, void* out, void* stream) {
  if (N < 0 || K < 0 || K % 32 || ldw < K || ((N > 0 && K > 0) && (!W || !out))) return PET_ATTN_EINVAL;
  if (reinterpret_cast<uintptr_t>(out) & 15) return PET_ATTN_EALIGN;
  return pet_gemm_pair_weights(W, N, K, ldw, false, out, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_linear_fused_smallk(int M, int N, int K, const float* A, int64_t lda, const void* Wpairs, float* C,
                                       int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                       int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!A || !Wpairs || !C || lda < K || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin, pre,
                                                                              ldpre, act)))
    return PET_ATTN_EINVAL;
  if (act == 2 && N % 2) return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  return pet_gemm_nt_sk(M, N, K, A, lda, Wpairs, C, ldc, e, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_linear_pair_rows(const float* X, int M, int K, int64_t ldx, void* out, void* stream) {
  if (M < 0 || K < 0 || ldx < K || (M > 0 && K > 0 && (!X || !out))) return PET_ATTN_EINVAL;
  return pet_gemm_pair_rows(X, M, K, ldx, out, reinterpret_cast<hipStream_t>(stream));
}

// the epilogue's operands for a product with no C (block pairs out)
static bool epi_args_nc_ok(int N, const float* row_scale, const float* cin, int64_t ldcin, const float* pre,
                           int64_t ldpre, int act) {
  if (act < 0 || act > 4) return false;
  if (act >= 3) return cin && ldcin >= (act == 4 ? 2 * int64_t(N) : N) && !row_scale && !pre;
  return (!cin || ldcin >= N) && (!pre || ldpre >= N);
}

extern "C" int pet_linear_fused_split_blocks(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit,
                                             void* out, const float* row_scale, const float* bias, const float* cin,
                                             int64_t ldcin, float beta, float* pre, int64_t ldpre, int act,
                                             void* scratch, size_t scratch_bytes, int* kb, void* stream) {
  if (!kb || (M > 0 && N > 0 && (!A || !Wsplit || !out || lda < K ||
                                  !epi_args_nc_ok(N, row_scale, cin, ldcin, pre, ldpre, act))))
    return PET_ATTN_EINVAL;
  return pet_gemm_nt_split_pairs(M, N, K, A, lda, Wsplit, out, row_scale, bias, cin, ldcin, beta, pre, ldpre, act,
                                 reinterpret_cast<hipStream_t>(stream), scratch, scratch_bytes, kb);
}

extern "C" int pet_linear_fused_blocks(int M, int N, int K, const void* Ablocks, int kb, const void* Wsplit, float* C,
                                       int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                       int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!Ablocks || !Wsplit || !C || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin, pre,
                                                                       ldpre, act)))
    return PET_ATTN_EINVAL;
  return pet_gemm_nt_pp_blocks(M, N, K, Ablocks, kb, Wsplit, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre,
                               act, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_linear_fused_pairs(int M, int N, int K, const void* Apairs, const void* Wsplit, float* C,
                                      int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                      int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream) {
  if ((M > 0 && N > 0) && (!Apairs || !Wsplit || !C || !epi_args_ok(N, C, ldc, row_scale, cin, ldcin, pre,
                                                                      ldpre, act)))
    return PET_ATTN_EINVAL;
  if (act == 2 && N % 2) return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
  return pet_gemm_nt_pp(M, N, K, Apairs, Wsplit, C, ldc, e, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pet_gemm_flop_tally(double* flops, int reset) {
  if (!flops) return PET_ATTN_EINVAL;
  for (int c = 0; c < 4; ++c)
    flops[c] = double(reset ? g_flops[c].exchange(0, std::memory_order_relaxed)
                            : g_flops[c].load(std::memory_order_relaxed));
  return PET_ATTN_OK;
}
