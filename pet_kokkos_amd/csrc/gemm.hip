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
};

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
  __shared__ u4 As[BM * RP], Bt[BN * RP];
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
__global__ void __launch_bounds__(64 * WGM * WGN) gemm_nt_pair_kernel(int M, int N, int K,
                                                                       const float* __restrict__ A, int64_t lda,
                                                                       const u4* __restrict__ Bs, float* C,
                                                                       int64_t ldc, Epi epi,
                                                                       const float* __restrict__ Bf, int64_t ldb,
                                                                       int cpw) {
  constexpr int T = 64 * WGM * WGN, NW = T / 64, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16, RP = 9;
  constexpr int AL = BM * 8 / T;  // float4 of a step's A slice, a thread's share
  constexpr int BL = BN * 8 / T;  // B slice: float4 (BF) or u4 slots, a thread's share
  static_assert(AL * T == BM * 8 && BL * T == BN * 8, "a step's slices divide evenly over the threads");
  __shared__ u4 As[BM * RP], Bt[BN * RP];
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
  epilogue<WM, WN>(acc, m0t, n0, wm, wn, c, g, M, N, C, ldc, epi);
  __syncthreads();  // the next tile's first slices overwrite this one's last
  }
}

// Rows of B = W (transposed false: W [N, K], ld ldw) or B = W^T (transposed
// true: W [K, N]) as fp16 pairs: out[(n K/8 + j) 2 + p] = part p (hi, lo) of
// row n's k group j, scaled by the row's s_n; then at byte N K 4 the N
// inverse scales 1 / s_n. One workgroup a row: its largest |x|, then its
// groups.
__global__ void __launch_bounds__(256) pair_rows_kernel(const float* __restrict__ W, int N, int K, int64_t ldw,
                                                         bool transposed, u4* __restrict__ out) {
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
    u4 hi, lo;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      unsigned h, lw;
      pair2(at(8 * j + 2 * e) * s, at(8 * j + 2 * e + 1) * s, h, lw);
      hi[e] = h, lo[e] = lw;
    }
    out[(int64_t(n) * KG + j) * 2] = hi;
    out[(int64_t(n) * KG + j) * 2 + 1] = lo;
  }
  if (tid == 0) reinterpret_cast<float*>(out + int64_t(N) * KG * 2)[n] = 1.f / s;
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

int pet_gemm_nt_split(int M, int N, int K, const float* A, int64_t lda, const void* Bs, float* C, int64_t ldc,
                      const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                      float* pre, int64_t ldpre, int act, hipStream_t st) {
  if (M < 0 || N < 0 || K < 0) return PET_ATTN_EINVAL;
  if (M == 0 || N == 0) return PET_ATTN_OK;
  if (K == 0) return PET_ATTN_EINVAL;
  if (int64_t((M + 63) / 64) * ((N + 63) / 64) >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;  // 1-D grid of tiles
  if (K % 32 || lda % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || (reinterpret_cast<uintptr_t>(Bs) & 15))
    return PET_ATTN_EALIGN;
  if (act == 2 && N % 2) return PET_ATTN_EINVAL;
  Epi e;
  e.row_scale = row_scale, e.bias = bias, e.cin = cin, e.ldcin = ldcin, e.beta = beta, e.pre = pre, e.ldpre = ldpre;
  e.act = act;
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
  };
  // measured on MI355X: 128 x 128 tiles of 8 waves where there are many
  // (131072 x 1536 x 512: 1200-1213 us against 1394-1418 for 128 x 64 and
  // 1535 for 64 x 64; 256 x 128 and 128 x 256 tiles of 16 waves were no
  // faster), 64 x 64 otherwise (27318 x 128 x 128: 16.1 against 18.4 us); one
  // LDS buffer beat two in every shape
  const int64_t t128 = int64_t((M + 127) / 128) * ((N + 63) / 64);
  if (pair_form(K)) {
    if (N >= 128 && t128 >= 2048)
      go(gemm_nt_pair_kernel<128, 128, 2, 4>, 128, 128, 512, true);
    else if (t128 >= 2048)
      go(gemm_nt_pair_kernel<128, 64>, 128, 64, 256, true);
    else
      go(gemm_nt_pair_kernel<64, 64>, 64, 64, 256, true);
  } else {
    if (N >= 128 && t128 >= 2048)
      go(gemm_nt_split_kernel<128, 128, 2, 4>, 128, 128, 512, false);
    else if (t128 >= 2048)
      go(gemm_nt_split_kernel<128, 64>, 128, 64, 256, false);
    else
      go(gemm_nt_split_kernel<64, 64>, 64, 64, 256, false);
  }
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
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
    hipLaunchKernelGGL(pair_rows_kernel, dim3(unsigned(N)), dim3(256), 0, st, W, N, K, ldw, transposed,
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
                           reinterpret_cast<hipStream_t>(stream));
}
