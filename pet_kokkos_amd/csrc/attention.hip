// PET's per-atom neighbourhood attention, forward and backward, for gfx950
// (MI355X), on the fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// Semantics follow the reference's attention()/attention_bwd()
// (peterspackman/pet-kokkos src/attention.cpp:1-16, :205-266, :1560-1697,
// :1814-1907): atom n's tokens are row n and rows N+off[n] .. N+off[n+1]-1 of
// the token matrix; per head, query i attends to key k with weight
// softmax_k(scale q_i.k_k + log cf_k); keys with cf <= 0 are left out and a
// query on a cf <= 0 edge yields zeros.
//
// Work decomposition (one workgroup per (atom, head)):
//   - the atom's head slices of K and V (backward: Q, K, V, dO) are staged in
//     LDS once, rows padded to 16-token blocks with zeros, pitch hd + 4 floats
//     so a 16-lane column of 128-bit reads touches distinct banks;
//   - wave w owns query block w (16 queries) -- and in the backward also key
//     block w -- for w < nb = ceil(count / 16); waves past nb only keep the
//     workgroup's barriers.
// MFMA lane layout, lane l = (c, g) = (l % 16, l / 16): operand a is A[c][g],
// operand b is B[g][c], and register r of the result is C[4g + r][c]. Scores
// are formed transposed (rows keys, columns queries), S^T = K Q^T, so a lane
// holds one query's scores against keys 4g + r: the softmax needs only
// cross-g reductions, and the weights are already the b operand of the next
// product O^T = V^T P^T. A lane's result rows are then dims
// (4g + r) * DT + t of its query (DT = hd / 16 tiles t), i.e. the contiguous
// slice [g hd/4, (g+1) hd/4): the same slice it loaded q from, written back
// with 128-bit stores.
//
// The backward never forms an S x S matrix in memory. At step s wave w forms
// the 16 x 16 tile (query block w, key block (w + s) mod nb): S^T and dP^T,
// then A and dS, adds its dQ share, and leaves A and dS in LDS; after one
// barrier the owner of that key block, wave (w + s) mod nb, takes the tile's
// dK, dV and cf shares. Every tile is computed once (the 10 cnt^2 hd flops of
// the algorithm, no recompute), each output has one owner summing in a fixed
// order, and nothing is atomic: the result is bit-identical run to run.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>

#include "../../include/pet_attn.h"

namespace pet_attn {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr float kOff = -1e30f;  // the log cf of a key no query sees
__device__ __forceinline__ bool is_off(float lc) { return lc < -1e29f; }

// Over the four lanes that share c (g = 0..3).
__device__ __forceinline__ float max_g(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float sum_g(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
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

// Geometry of one atom's tokens.
struct Atom {
  int n, N, o0, cnt, nb;
  __device__ Atom(const int* off, int n_, int N_, int S) : n(n_), N(N_) {
    o0 = off[n];
    const int c = off[n + 1] - o0 + 1;
    cnt = c < S ? c : S;  // a count above S would be the caller's error; never read past S
    nb = (cnt + 15) >> 4;
  }
  __device__ size_t row(int s) const { return s == 0 ? size_t(n) : size_t(N) + size_t(o0) + size_t(s - 1); }
};

// Rows [0, nb*16) of the atom's head slice at column `col` of src into dst
// (pitch P), zero past the count.
template <int HD, int P>
__device__ __forceinline__ void stage_rows(float* dst, const float* src, int64_t ld, int col, const Atom& at) {
  constexpr int C4 = HD / 4;
  const int total = at.nb * 16 * C4;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int r = idx / C4, c4 = idx - r * C4;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < at.cnt) x = *reinterpret_cast<const float4*>(src + at.row(r) * ld + col + 4 * c4);
    *reinterpret_cast<float4*>(dst + r * P + 4 * c4) = x;
  }
}
__device__ __forceinline__ void stage_log_cf(float* lcf, const float* cf, const Atom& at) {
  for (int r = threadIdx.x; r < at.nb * 16; r += blockDim.x) {
    float lc = kOff;
    if (r < at.cnt) {
      const float c = cf[r];
      lc = c > 0.f ? __logf(c) : kOff;
    }
    lcf[r] = lc;
  }
}

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

template <int HD>
struct Lds {
  static constexpr int P = HD + 4;   // row pitch of staged slices
  static constexpr int TP = 16 + 4;  // row pitch of a 16 x 16 tile
  static size_t fwd_floats(int NW) { return size_t(2) * NW * 16 * P + NW * 16; }
  static size_t bwd_floats(int NW) { return size_t(4) * NW * 16 * P + NW * 16 + size_t(2) * NW * 2 * 16 * TP; }
};

// ---- forward ---------------------------------------------------------------
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_fwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int S, int H, float sc,
                                                        const float* __restrict__ cf_seq, int64_t ldc,
                                                        float* __restrict__ merged, int64_t ldm,
                                                        float* __restrict__ ml) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6;
  const int n = blockIdx.x / H, h = blockIdx.x - n * H, D = H * HD;
  const Atom at(off, n, N, S);
  float* Ks = lds;
  float* Vs = Ks + NW * 16 * P;
  float* lcf = Vs + NW * 16 * P;
  stage_rows<HD, P>(Ks, qkv, ldq, D + h * HD, at);
  stage_rows<HD, P>(Vs, qkv, ldq, 2 * D + h * HD, at);
  stage_log_cf(lcf, cf_seq + size_t(n) * ldc, at);
  __syncthreads();

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;  // this lane's query slot
  float* mlq = ml ? ml + 2 * ((size_t(n) * H + h) * S + i) : nullptr;
  if (w >= at.nb) {  // slots past the atom's tokens: no rows
    if (mlq && g == 0 && i < S) mlq[0] = kOff, mlq[1] = 0.f;
    return;
  }
  float q[W];
  if (i < at.cnt)
    gmem_get<W>(qkv + at.row(i) * ldq + h * HD + g * W, q);
  else
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = 0.f;

  float mx = kOff, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  for (int J = 0; J < at.nb; ++J) {
    float k[W];
    lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
    f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);  // s[r]: query i, key 16J + 4g + r
    float lc[4];
    lds_get<4>(lcf + 16 * J + 4 * g, lc);
    float x[4], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = is_off(lc[r]) ? kOff : s[r] * sc + lc[r];
      bm = fmaxf(bm, x[r]);
    }
    const float nm = fmaxf(mx, max_g(bm));
    const float alpha = __expf(mx - nm);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = is_off(lc[r]) ? 0.f : __expf(x[r] - nm);
    sum = sum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    mx = nm;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v[DT];
      lds_get<DT>(Vs + (16 * J + 4 * g + r) * P + c * DT, v);
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] = mfma(v[t], p[r], acc[t]);  // O^T: dim (4g + r') DT + t, query i
    }
  }
  const float tot = sum_g(sum);
  if (i >= S) return;
  if (i >= at.cnt) {  // a slot past the atom's tokens
    if (mlq && g == 0) mlq[0] = kOff, mlq[1] = 0.f;
    return;
  }
  const bool live = i == 0 || !is_off(lcf[i]);  // else a query on an edge at its cutoff: zeros
  const float invl = live && tot > 0.f ? 1.0f / tot : 0.f;
  store_slice<HD>(merged + at.row(i) * ldm + h * HD + g * W, acc, invl);
  if (mlq && g == 0) mlq[0] = live ? mx : kOff, mlq[1] = invl;
}

// ---- backward --------------------------------------------------------------
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_bwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int S, int H, float sc,
                                                        const float* __restrict__ dmerged, int64_t ldg,
                                                        const float* __restrict__ merged, int64_t ldm,
                                                        const float* __restrict__ ml,
                                                        const float* __restrict__ cf_seq, int64_t ldc,
                                                        float* __restrict__ qkv_adj, int64_t lda,
                                                        float* __restrict__ cfh) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P, TP = Lds<HD>::TP, TILE = 16 * TP;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16;
  const int n = blockIdx.x / H, h = blockIdx.x - n * H, D = H * HD;
  const Atom at(off, n, N, S);
  float* Qs = lds;
  float* Ks = Qs + R * P;
  float* Vs = Ks + R * P;
  float* Gs = Vs + R * P;
  float* lcf = Gs + R * P;
  float* Tb = lcf + R;  // [2 buffers][NW producers][A, dS][16 x TP]
  stage_rows<HD, P>(Qs, qkv, ldq, h * HD, at);
  stage_rows<HD, P>(Ks, qkv, ldq, D + h * HD, at);
  stage_rows<HD, P>(Vs, qkv, ldq, 2 * D + h * HD, at);
  stage_rows<HD, P>(Gs, dmerged, ldg, h * HD, at);
  stage_log_cf(lcf, cf_seq + size_t(n) * ldc, at);

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bool active = w < at.nb;
  const int i = 16 * w + c;  // this lane's query slot, and its key slot
  float mi = kOff, li = 0.f, dqi = 0.f;
  if (active) {
    float go[W], oo[W];
    if (i < at.cnt) {
      gmem_get<W>(dmerged + at.row(i) * ldg + h * HD + g * W, go);
      gmem_get<W>(merged + at.row(i) * ldm + h * HD + g * W, oo);
    } else {
#pragma unroll
      for (int t = 0; t < W; ++t) go[t] = oo[t] = 0.f;
    }
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < W; ++t) d += go[t] * oo[t];
    dqi = sum_g(d);  // Dq = dO . O of query i
    if (i < at.cnt) {
      const float* m2 = ml + 2 * ((size_t(n) * H + h) * S + i);
      mi = m2[0], li = m2[1];
    }
  }
  __syncthreads();

  float q[W], go[W];
  if (active) {
    lds_get<W>(Qs + i * P + g * W, q);
    lds_get<W>(Gs + i * P + g * W, go);
  }
  f4 dq[DT], dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  const int nb = at.nb;
  for (int s = 0; s < nb; ++s) {
    float* tb = Tb + (s & 1) * (NW * 2 * TILE);
    if (active) {
      // Tile (query block w, key block J): S^T and dP^T, then A and dS.
      int J = w + s;
      if (J >= nb) J -= nb;
      f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
      {
        float k[W], v[W];
        lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
        lds_get<W>(Vs + (16 * J + c) * P + g * W, v);
#pragma unroll
        for (int t = 0; t < W; ++t) st = mfma(k[t], q[t], st), dp = mfma(v[t], go[t], dp);
      }
      float lc[4], a[4], ds[4];
      lds_get<4>(lcf + 16 * J + 4 * g, lc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // query i, key 16J + 4g + r
        a[r] = li > 0.f && !is_off(lc[r]) ? __expf(st[r] * sc + lc[r] - mi) * li : 0.f;
        ds[r] = a[r] * (dp[r] - dqi);
      }
      // dQ^T += K^T dS^T over the tile's keys.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float kk[DT];
        lds_get<DT>(Ks + (16 * J + 4 * g + r) * P + c * DT, kk);
#pragma unroll
        for (int t = 0; t < DT; ++t) dq[t] = mfma(kk[t], ds[r], dq[t]);
      }
      float* ta = tb + (2 * w) * TILE;
      *reinterpret_cast<float4*>(ta + c * TP + 4 * g) = make_float4(a[0], a[1], a[2], a[3]);
      *reinterpret_cast<float4*>(ta + TILE + c * TP + 4 * g) = make_float4(ds[0], ds[1], ds[2], ds[3]);
    }
    __syncthreads();
    if (active) {
      // Key block w's tile from query block Ip: dK^T += Q^T dS, dV^T += dO^T A.
      int Ip = w - s;
      if (Ip < 0) Ip += nb;
      const float* ta = tb + (2 * Ip) * TILE;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float av = ta[(4 * g + r) * TP + c], dsv = ta[TILE + (4 * g + r) * TP + c];
        cfa += dsv;
        float qq[DT], gg[DT];
        lds_get<DT>(Qs + (16 * Ip + 4 * g + r) * P + c * DT, qq);
        lds_get<DT>(Gs + (16 * Ip + 4 * g + r) * P + c * DT, gg);
#pragma unroll
        for (int t = 0; t < DT; ++t) dk[t] = mfma(qq[t], dsv, dk[t]), dv[t] = mfma(gg[t], av, dv[t]);
      }
    }
  }
  const float cft = sum_g(cfa);
  if (active && i < at.cnt) {
    float* o = qkv_adj + at.row(i) * lda + h * HD + g * W;
    store_slice<HD>(o, dq, sc);
    store_slice<HD>(o + D, dk, sc);
    store_slice<HD>(o + 2 * D, dv, 1.0f);
  }
  if (g == 0 && i < S) cfh[(size_t(n) * S + i) * H + h] = active && i < at.cnt ? cft : 0.f;
}

// cf_seq_adj(n, k) += sum_h cfh(n S + k, h) / cf(n, k) where cf > 0, heads in
// order (the reference's attn_bwd_cf, src/attention.cpp:1829-1838).
__global__ void attn_cf_adjoint_kernel(const float* __restrict__ cfh, const float* __restrict__ cf_seq, int64_t ldc,
                                       float* __restrict__ cf_seq_adj, int64_t ldca, int N, int S, int H) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(N) * S) return;
  const int n = int(i / S), k = int(i - int64_t(n) * S);
  const float cf = cf_seq[int64_t(n) * ldc + k];
  if (cf <= 0.f) return;
  float total = 0.f;
  for (int hh = 0; hh < H; ++hh) total += cfh[i * H + hh];
  cf_seq_adj[int64_t(n) * ldca + k] += total / cf;
}

// A capacity's dead rows, N + off[N] .. T-1, of x[T, width] set to zero
// (the reference's zero_dead, src/attention.cpp:1510-1518).
__global__ void zero_dead_kernel(float* __restrict__ x, int64_t ld, int width, int N, int T,
                                 const int* __restrict__ off) {
  const int64_t first = int64_t(N) + off[N];
  const int64_t total = (int64_t(T) - N) * width;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = N + i / width;
    if (r >= first) x[r * ld + (i % width)] = 0.f;
  }
}

// ---- host side ---------------------------------------------------------------

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int max_lds_bytes() {
  static int bytes = [] {
    int dev = 0, b = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 65536;
    if (hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 65536;
    return b;
  }();
  return bytes;
}

int check_shape(const pet_attn_shape* sh) {
  if (!sh) return PET_ATTN_EINVAL;
  if (sh->n_atoms < 0 || sh->n_rows < sh->n_atoms || sh->slots < 1 || sh->heads < 1) return PET_ATTN_EINVAL;
  if (sh->head_dim < 16 || sh->head_dim > 128 || sh->head_dim % 16 != 0) return PET_ATTN_EHEADDIM;
  if (sh->slots > PET_ATTN_MAX_SLOTS) return PET_ATTN_ESLOTS;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (int64_t(sh->n_rows) * 3 * D >= (int64_t(1) << 31) * 4) return PET_ATTN_EINDEX;
  if (int64_t(sh->n_atoms) * sh->heads * sh->slots >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  if (int64_t(sh->n_atoms) * sh->heads >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  return PET_ATTN_OK;
}
int check_matrix(const void* p, int64_t ld, int64_t width) {
  if (!p || ld < width) return PET_ATTN_EINVAL;
  if (!aligned16(p) || ld % 4 != 0) return PET_ATTN_EALIGN;
  return PET_ATTN_OK;
}
int waves_for(int S) { return (S + 15) / 16; }

template <int HD>
int launch_fwd(const pet_attn_shape& sh, const float* qkv, int64_t ldq, const int* off, const float* cf_seq,
               int64_t ldc, float* merged, int64_t ldm, float* ml, hipStream_t st) {
  const int NW = waves_for(sh.slots);
  const size_t bytes = sizeof(float) * Lds<HD>::fwd_floats(NW);
  if (bytes > size_t(max_lds_bytes())) return PET_ATTN_ESLOTS;
  const dim3 grid(unsigned(sh.n_atoms) * sh.heads), block(64 * NW);
  if (NW <= 8) {
    auto k = attn_fwd_kernel<HD, 512>;
    if (bytes > 65536) (void) hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    hipLaunchKernelGGL(k, grid, block, bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                       cf_seq, ldc, merged, ldm, ml);
  } else {
    auto k = attn_fwd_kernel<HD, 1024>;
    if (bytes > 65536) (void) hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    hipLaunchKernelGGL(k, grid, block, bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                       cf_seq, ldc, merged, ldm, ml);
  }
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

template <int HD>
int launch_bwd(const pet_attn_shape& sh, const float* qkv, int64_t ldq, const int* off, const float* dmerged,
               int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
               float* qkv_adj, int64_t lda, float* cfh, hipStream_t st) {
  const int NW = waves_for(sh.slots);
  const size_t bytes = sizeof(float) * Lds<HD>::bwd_floats(NW);
  if (bytes > size_t(max_lds_bytes())) return PET_ATTN_ESLOTS;
  const dim3 grid(unsigned(sh.n_atoms) * sh.heads), block(64 * NW);
  if (NW <= 8) {
    auto k = attn_bwd_kernel<HD, 512>;
    if (bytes > 65536) (void) hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    hipLaunchKernelGGL(k, grid, block, bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                       dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh);
  } else {
    auto k = attn_bwd_kernel<HD, 1024>;
    if (bytes > 65536) (void) hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    hipLaunchKernelGGL(k, grid, block, bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                       dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh);
  }
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

template <class F>
int with_head_dim(int hd, F&& f) {
  switch (hd) {
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 48: return f(std::integral_constant<int, 48>{});
    case 64: return f(std::integral_constant<int, 64>{});
    case 80: return f(std::integral_constant<int, 80>{});
    case 96: return f(std::integral_constant<int, 96>{});
    case 112: return f(std::integral_constant<int, 112>{});
    case 128: return f(std::integral_constant<int, 128>{});
    default: return PET_ATTN_EHEADDIM;
  }
}

int zero_dead(float* x, int64_t ld, int width, const pet_attn_shape& sh, const int* off, hipStream_t st) {
  if (!sh.dead || sh.n_rows == sh.n_atoms) return PET_ATTN_OK;
  const int64_t total = (int64_t(sh.n_rows) - sh.n_atoms) * width;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(zero_dead_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, x, ld,
                     width, sh.n_atoms, sh.n_rows, off);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

}  // namespace pet_attn

using namespace pet_attn;

extern "C" {

float pet_attn_scale(int head_dim, double temperature) {
  return float(1.0 / (std::sqrt(double(head_dim)) * temperature));
}

const char* pet_attn_strerror(int code) {
  switch (code) {
    case PET_ATTN_OK: return "ok";
    case PET_ATTN_EINVAL: return "invalid argument (null pointer, negative size or leading dimension too small)";
    case PET_ATTN_EHEADDIM: return "unsupported head_dim (a multiple of 16, at most 128)";
    case PET_ATTN_ESLOTS: return "too many slots per atom for the kernels' LDS (at most 256, less for wide heads)";
    case PET_ATTN_EALIGN: return "a pointer or leading dimension is not a multiple of 4 floats";
    case PET_ATTN_ELAUNCH: return "a HIP launch or runtime call failed";
    case PET_ATTN_EBLAS: return "the BLAS call of a linear failed";
    case PET_ATTN_EWORKSPACE: return "workspace smaller than pet_attention_bwd_workspace()";
    case PET_ATTN_EINDEX: return "an index does not fit 2^31";
    default: return "unknown pet_attn error";
  }
}

int pet_attn_fwd(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* cf_seq,
                 int64_t ldc, float* merged, int64_t ldm, float* ml, void* stream) {
  if (int e = check_shape(sh)) return e;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  if (int e = check_matrix(qkv, ldq, 3 * D)) return e;
  if (int e = check_matrix(merged, ldm, D)) return e;
  if (!off || !cf_seq || ldc < sh->slots) return PET_ATTN_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int e = with_head_dim(sh->head_dim, [&](auto hd) {
    return launch_fwd<decltype(hd)::value>(*sh, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, st);
  });
  if (e) return e;
  return zero_dead(merged, ldm, int(D), *sh, off, st);
}

int pet_attn_bwd(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* dmerged,
                 int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
                 float* qkv_adj, int64_t lda, float* cfh, float* cf_seq_adj, int64_t ldca, void* stream) {
  if (int e = check_shape(sh)) return e;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  if (int e = check_matrix(qkv, ldq, 3 * D)) return e;
  if (int e = check_matrix(dmerged, ldg, D)) return e;
  if (int e = check_matrix(merged, ldm, D)) return e;
  if (int e = check_matrix(qkv_adj, lda, 3 * D)) return e;
  if (!off || !ml || !cf_seq || !cfh || !cf_seq_adj || ldc < sh->slots || ldca < sh->slots) return PET_ATTN_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int e = with_head_dim(sh->head_dim, [&](auto hd) {
    return launch_bwd<decltype(hd)::value>(*sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj,
                                           lda, cfh, st);
  });
  if (e) return e;
  const int64_t NS = int64_t(sh->n_atoms) * sh->slots;
  hipLaunchKernelGGL(attn_cf_adjoint_kernel, dim3(unsigned((NS + 255) / 256)), dim3(256), 0, st, cfh, cf_seq, ldc,
                     cf_seq_adj, ldca, sh->n_atoms, sh->slots, sh->heads);
  if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
  return zero_dead(qkv_adj, lda, int(3 * D), *sh, off, st);
}

}  // extern "C"
