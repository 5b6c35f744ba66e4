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
#include <cstdlib>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/pet_attn.h"

namespace pet_attn {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr float kOff = -1e30f;  // the log cf of a key no query sees
__device__ __forceinline__ bool is_off(float lc) { return lc < -1e29f; }

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

// One work item, an (atom, head): the atom's token count and rows.
struct Atom {
  int n, h, N, o0, cnt, nb;
  __device__ Atom(const int* off, int item, int H, int N_, int S) : N(N_) {
    n = item / H;
    h = item - n * H;
    o0 = off[n];
    const int c = off[n + 1] - o0 + 1;
    cnt = c < S ? c : S;  // a count above S would be the caller's error; never read past S
    nb = (cnt + 15) >> 4;
  }
  __device__ size_t row(int s) const { return s == 0 ? size_t(n) : size_t(N) + size_t(o0) + size_t(s - 1); }
};

// A thread's share of one head slice of an item's rows [0, 16 NW), held in
// registers between its global load (issued while the previous item is
// computed) and its store to LDS: blockDim = 64 NW threads, hd/16 float4 each.
template <int HD>
struct SliceRegs {
  static constexpr int C4 = HD / 4, PER = HD / 16;
  float4 v[PER];
  __device__ __forceinline__ void load(const float* src, int64_t ld, int col, const Atom& at) {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int idx = threadIdx.x + k * blockDim.x, r = idx / C4, c4 = idx - r * C4;
      v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r < at.cnt) v[k] = *reinterpret_cast<const float4*>(src + at.row(r) * ld + col + 4 * c4);
    }
  }
  template <int P>
  __device__ __forceinline__ void store(float* dst) const {
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int idx = threadIdx.x + k * blockDim.x, r = idx / C4, c4 = idx - r * C4;
      *reinterpret_cast<float4*>(dst + r * P + 4 * c4) = v[k];
    }
  }
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

template <int HD>
struct Lds {
  static constexpr int P = HD + 4;   // row pitch of staged slices
  static constexpr int TP = 16 + 4;  // row pitch of a 16 x 16 tile
  static size_t fwd_floats(int NW) { return size_t(2) * NW * 16 * P + NW * 16; }
  // nbuf tile buffers: 2 lets a step's producers write while the last step's
  // owners still read (one barrier a step); 1 needs two barriers a step.
  // vlds: V staged too (else its rows come from global memory).
  static size_t bwd_floats(int NW, int nbuf, bool vlds) {
    return size_t(vlds ? 4 : 3) * NW * 16 * P + NW * 16 + size_t(nbuf) * NW * 2 * 16 * TP;
  }
};

// ---- forward ---------------------------------------------------------------
// A lane's share of one item's forward result, held until it is stored.
template <int HD>
struct FwdOut {
  f4 acc[HD / 16];
  float mx, invl;
  bool live;
};

// One item's forward from the staged K, V and log cf: wave w, query block w.
template <int HD>
__device__ __forceinline__ void fwd_item(const Atom& at, const float* Ks, const float* Vs, const float* lcf,
                                         const float* q, float sc, FwdOut<HD>& out) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;  // this lane's query slot
  if (w >= at.nb) return;    // slots past the atom's tokens
  float mx = kOff, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  // S^T of key block J: s[r] = query i against key 16J + 4g + r.
  auto scores = [&](int J) {
    float k[W];
    lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
    f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);
    return s;
  };
  // Online softmax and PV of key block J from its scores s.
  auto block = [&](int J, const f4& s) {
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
  };
  // The next block's scores go out before this block's softmax and PV, in
  // one basic block the scheduler interleaves; the last block is peeled.
  f4 s = scores(0);
  for (int J = 0; J + 1 < at.nb; ++J) {
    const f4 sn = scores(J + 1);
    block(J, s);
    s = sn;
  }
  block(at.nb - 1, s);
  const float tot = sum_g(sum);
  // else a query on an edge at its cutoff: zeros
  out.live = i < at.cnt && (i == 0 || !is_off(lcf[i]));
  out.invl = out.live && tot > 0.f ? 1.0f / tot : 0.f;
  out.mx = out.live ? mx : kOff;
#pragma unroll
  for (int t = 0; t < DT; ++t) out.acc[t] = acc[t];
}

// The item's stores: merged rows of its tokens, ml of its S slots.
template <int HD>
__device__ __forceinline__ void fwd_store(const Atom& at, const FwdOut<HD>& out, int S, int H,
                                          float* __restrict__ merged, int64_t ldm, float* __restrict__ ml) {
  constexpr int W = HD / 4;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;
  if (i >= S) return;
  if (w < at.nb && i < at.cnt) store_slice<HD>(merged + at.row(i) * ldm + at.h * HD + g * W, out.acc, out.invl);
  if (ml && g == 0) {
    float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    const bool real = w < at.nb && i < at.cnt;
    mlq[0] = real ? out.mx : kOff, mlq[1] = real ? out.invl : 0.f;
  }
}

// Persistent: workgroup b takes items b, b + gridDim.x, ...; while it computes
// one, its threads' loads of the next are in flight, and its stores are issued
// after the next item's loads have landed (on gfx9 the memory counter a load
// waits on also counts earlier stores).
template <int HD>
__device__ __forceinline__ void attn_fwd_kernel_body(const float* __restrict__ qkv, int64_t ldq,
                                                     const int* __restrict__ off, int N, int S, int H, float sc,
                                                     const float* __restrict__ cf_seq, int64_t ldc,
                                                     float* __restrict__ merged, int64_t ldm,
                                                     float* __restrict__ ml) {
  constexpr int W = HD / 4, P = Lds<HD>::P;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD, items = N * H;
  float* Ks = lds;
  float* Vs = Ks + R * P;
  float* lcf = Vs + R * P;
  const int l = threadIdx.x & 63, g = l >> 4, i = 16 * (threadIdx.x >> 6) + (l & 15);
  int item = blockIdx.x;
  if (item >= items) return;
  Atom at(off, item, H, N, S);
  SliceRegs<HD> pk, pv;
  float pcf, pq[W];
  auto fetch = [&](const Atom& a) {
    pk.load(qkv, ldq, D + a.h * HD, a);
    pv.load(qkv, ldq, 2 * D + a.h * HD, a);
    pcf = int(threadIdx.x) < a.cnt ? cf_seq[size_t(a.n) * ldc + threadIdx.x] : 0.f;
    if (i < a.cnt)
      gmem_get<W>(qkv + a.row(i) * ldq + a.h * HD + g * W, pq);
    else
#pragma unroll
      for (int t = 0; t < W; ++t) pq[t] = 0.f;
  };
  fetch(at);
  FwdOut<HD> out;
  Atom done = at;
  bool pending = false;
  for (;;) {
    pk.template store<P>(Ks);
    pv.template store<P>(Vs);
    if (int(threadIdx.x) < R) lcf[threadIdx.x] = pcf > 0.f ? __logf(pcf) : kOff;
    float q[W];
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = pq[t];
    if (pending) fwd_store<HD>(done, out, S, H, merged, ldm, ml);
    const Atom cur = at;
    lds_barrier();
    const int next = item + gridDim.x;
    if (next < items) {
      at = Atom(off, next, H, N, S);
      fetch(at);
    }
    fwd_item<HD>(cur, Ks, Vs, lcf, q, sc, out);
    done = cur;
    pending = true;
    if (next >= items) break;
    lds_barrier();
    item = next;
  }
  fwd_store<HD>(done, out, S, H, merged, ldm, ml);
}
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_fwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int S, int H, float sc,
                                                        const float* __restrict__ cf_seq, int64_t ldc,
                                                        float* __restrict__ merged, int64_t ldm,
                                                        float* __restrict__ ml) {
  attn_fwd_kernel_body<HD>(qkv, ldq, off, N, S, H, sc, cf_seq, ldc, merged, ldm, ml);
}

// One item per workgroup: the item's K, V and q loaded into registers, staged
// in LDS, one barrier, then its forward.
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_fwd1_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int S, int H, float sc,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ merged, int64_t ldm,
                                                         float* __restrict__ ml) {
  constexpr int W = HD / 4, P = Lds<HD>::P;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD;
  float* Ks = lds;
  float* Vs = Ks + R * P;
  float* lcf = Vs + R * P;
  const int l = threadIdx.x & 63, g = l >> 4, i = 16 * (threadIdx.x >> 6) + (l & 15);
  const Atom at(off, blockIdx.x, H, N, S);
  float q[W];
  {
    SliceRegs<HD> pk, pv;
    pk.load(qkv, ldq, D + at.h * HD, at);
    pv.load(qkv, ldq, 2 * D + at.h * HD, at);
    const float pcf = int(threadIdx.x) < at.cnt ? cf_seq[size_t(at.n) * ldc + threadIdx.x] : 0.f;
    if (i < at.cnt)
      gmem_get<W>(qkv + at.row(i) * ldq + at.h * HD + g * W, q);
    else
#pragma unroll
      for (int t = 0; t < W; ++t) q[t] = 0.f;
    pk.template store<P>(Ks);
    pv.template store<P>(Vs);
    if (int(threadIdx.x) < R) lcf[threadIdx.x] = pcf > 0.f ? __logf(pcf) : kOff;
  }
  lds_barrier();
  FwdOut<HD> out;
  fwd_item<HD>(at, Ks, Vs, lcf, q, sc, out);
  fwd_store<HD>(at, out, S, H, merged, ldm, ml);
}

// No LDS and no barrier: each wave streams its atom's 16-key blocks of K and
// V straight from memory (the workgroup's waves share them through L1/L2),
// loading block J + 1 while it works on block J.
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_fwd2_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int S, int H, float sc,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ merged, int64_t ldm,
                                                         float* __restrict__ ml) {
  constexpr int W = HD / 4, DT = HD / 16;
  const int D = H * HD;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4, i = 16 * w + c;
  const Atom at(off, blockIdx.x, H, N, S);
  FwdOut<HD> out;
  if (w >= at.nb) {
    fwd_store<HD>(at, out, S, H, merged, ldm, ml);
    return;
  }
  const float* K = qkv + D + at.h * HD;
  const float* V = qkv + 2 * D + at.h * HD;
  const float* cf = cf_seq + size_t(at.n) * ldc;
  float q[W];
  if (i < at.cnt)
    gmem_get<W>(qkv + at.row(i) * ldq + at.h * HD + g * W, q);
  else
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = 0.f;
  float kn[W], vn[4][DT], cn[4];
  auto fetch = [&](int J) {
    const int rk = 16 * J + c;
    if (rk < at.cnt)
      gmem_get<W>(K + at.row(rk) * ldq + g * W, kn);
    else
#pragma unroll
      for (int t = 0; t < W; ++t) kn[t] = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int rv = 16 * J + 4 * g + r;
      cn[r] = rv < at.cnt ? cf[rv] : 0.f;
#pragma unroll
      for (int t = 0; t < DT; ++t) vn[r][t] = 0.f;
      if (rv < at.cnt) {
        const float* vp = V + at.row(rv) * ldq + c * DT;
#pragma unroll
        for (int t = 0; t < DT; ++t) vn[r][t] = vp[t];
      }
    }
  };
  fetch(0);
  float mx = kOff, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  for (int J = 0; J < at.nb; ++J) {
    float k[W], v[4][DT], lc[4];
#pragma unroll
    for (int t = 0; t < W; ++t) k[t] = kn[t];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      lc[r] = cn[r] > 0.f ? __logf(cn[r]) : kOff;
#pragma unroll
      for (int t = 0; t < DT; ++t) v[r][t] = vn[r][t];
    }
    if (J + 1 < at.nb) fetch(J + 1);
    f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);
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
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] = mfma(v[r][t], p[r], acc[t]);
  }
  const float tot = sum_g(sum);
  out.live = i < at.cnt && (i == 0 || cf[i] > 0.f);
  out.invl = out.live && tot > 0.f ? 1.0f / tot : 0.f;
  out.mx = out.live ? mx : kOff;
#pragma unroll
  for (int t = 0; t < DT; ++t) out.acc[t] = acc[t];
  fwd_store<HD>(at, out, S, H, merged, ldm, ml);
}

// The persistent forward held to 8 waves a SIMD (64 registers a lane).
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(8, 8)))
attn_fwd3_kernel(const float* __restrict__ qkv, int64_t ldq, const int* __restrict__ off, int N, int S, int H,
                 float sc, const float* __restrict__ cf_seq, int64_t ldc, float* __restrict__ merged, int64_t ldm,
                 float* __restrict__ ml) {
  attn_fwd_kernel_body<HD>(qkv, ldq, off, N, S, H, sc, cf_seq, ldc, merged, ldm, ml);
}

// ---- forward, LDS-DMA pipelined ------------------------------------------------
// gfx950 loads global memory straight into LDS (global_load_lds_dwordx4: lane
// l of a wave writes 16 bytes at base + 16 l), no registers in between. A
// persistent workgroup keeps two item buffers: while it computes item k from
// one, item k + 1's rows stream into the other.
//
// A buffer holds the item's K and V slices interleaved, one 2 hd-float row
// per token slot (16 NW rows), then the slots' raw cutoff factors. Row r's
// float4 q of the K half (0 <= q < hd/4) sits at slot q ^ (r & M), of the V
// half at hd/4 + (q ^ (r & M)), M + 1 the largest power of two <= 8 dividing
// hd/4: the MFMA operand reads -- 16 rows at one column, or one row's 16
// columns -- then touch distinct banks. Slots past the atom's count load its
// own row (finite values) and are masked by index.
typedef __attribute__((address_space(1))) const void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;

template <int HD>
struct KV {
  static constexpr int C4 = HD / 4;                 // float4 per half row
  static constexpr int RQ = 2 * C4;                 // float4 per row
  static constexpr int M = (C4 % 8 == 0) ? 7 : 3;   // swizzle mask (C4 is a multiple of 4)
  static constexpr int RF = 4 * RQ;                 // floats per row
  __host__ __device__ static size_t floats(int NW) { return size_t(16) * NW * RF + 16 * NW; }  // rows + cf
  // Float index of logical float x (0 <= x < 2 hd: K then V) of row r.
  __device__ static __forceinline__ int at(int r, int x) {
    const int q = x >> 2, half = q >= C4 ? C4 : 0, qq = q - half;
    return r * RF + 4 * (half + (qq ^ (r & M))) + (x & 3);
  }
};

// Issue the LDS-DMA loads of one item into buffer `buf` (all threads).
template <int HD>
__device__ __forceinline__ void kv_issue(float* buf, const float* __restrict__ qkv, int64_t ldq, int D,
                                         const float* __restrict__ cf_seq, int64_t ldc, const Atom& at) {
  constexpr int RQ = KV<HD>::RQ, C4 = KV<HD>::C4, M = KV<HD>::M;
  const int NW = blockDim.x >> 6, w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int chunks = NW * 16 * RQ / 64;  // 1 KB chunks of the row block
  for (int j = w; j < chunks; j += NW) {
    const int f = 64 * j + l, r = f / RQ, p = f - r * RQ;  // physical float4 slot p of row r
    const int half = p >= C4 ? C4 : 0, q = (p - half) ^ (r & M);
    const int src = r < at.cnt ? r : 0;
    const float* g = qkv + at.row(src) * ldq + (half ? 2 * D : D) + at.h * HD + 4 * q;
    __builtin_amdgcn_global_load_lds((gvoid_t*) g, (lvoid_t*) (buf + 256 * j), 16, 0, 0);
  }
  // the cf of slots 0 .. 16 NW - 1 (slots past the count read slot 0's)
  float* cfb = buf + NW * 16 * KV<HD>::RF;
  for (int j = w; j * 64 < NW * 16; j += NW) {
    const int sl = 64 * j + l;
    if (sl < NW * 16)
      __builtin_amdgcn_global_load_lds((gvoid_t*) (cf_seq + size_t(at.n) * ldc + (sl < at.cnt ? sl : 0)),
                                       (lvoid_t*) (cfb + 64 * j), 4, 0, 0);
  }
}

__device__ __forceinline__ void wait_vm_all() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), other counters free
}

// One item's forward from a KV buffer: wave w, query block w.
template <int HD>
__device__ __forceinline__ void fwd_item_kv(const Atom& at, const float* buf, const float* q, float sc,
                                            FwdOut<HD>& out) {
  constexpr int W = HD / 4, DT = HD / 16, RF = KV<HD>::RF, M = KV<HD>::M, C4 = KV<HD>::C4;
  const int NW = blockDim.x >> 6;
  const float* cfb = buf + NW * 16 * RF;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;
  if (w >= at.nb) return;
  float mx = kOff, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  for (int J = 0; J < at.nb; ++J) {
    const int rk = 16 * J + c;
    float k[W];
#pragma unroll
    for (int u = 0; u < W / 4; ++u) {
      const float4 x = *reinterpret_cast<const float4*>(buf + rk * RF + 4 * ((g * (W / 4) + u) ^ (rk & M)));
      k[4 * u] = x.x, k[4 * u + 1] = x.y, k[4 * u + 2] = x.z, k[4 * u + 3] = x.w;
    }
    f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);  // s[r]: query i, key 16J + 4g + r
    const float4 cf4 = *reinterpret_cast<const float4*>(cfb + 16 * J + 4 * g);
    const float cfr[4] = {cf4.x, cf4.y, cf4.z, cf4.w};
    float lc[4], x[4], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = 16 * J + 4 * g + r;
      lc[r] = key < at.cnt && cfr[r] > 0.f ? __logf(cfr[r]) : kOff;
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
      const int rv = 16 * J + 4 * g + r;
      float v[DT];
      if constexpr (DT == 2 || DT == 4) {
        // DT consecutive floats inside one float4 of the V half
        const int x0 = c * DT, qv = x0 >> 2;
        const float* pv = buf + rv * RF + 4 * (C4 + (qv ^ (rv & M))) + (x0 & 3);
        if constexpr (DT == 4) {
          const float4 y = *reinterpret_cast<const float4*>(pv);
          v[0] = y.x, v[1] = y.y, v[2] = y.z, v[3] = y.w;
        } else {
          const float2 y = *reinterpret_cast<const float2*>(pv);
          v[0] = y.x, v[1] = y.y;
        }
      } else {
#pragma unroll
        for (int t = 0; t < DT; ++t) v[t] = buf[KV<HD>::at(rv, HD + c * DT + t)];
      }
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] = mfma(v[t], p[r], acc[t]);
    }
  }
  const float tot = sum_g(sum);
  out.live = i < at.cnt && (i == 0 || cfb[i] > 0.f);
  out.invl = out.live && tot > 0.f ? 1.0f / tot : 0.f;
  out.mx = out.live ? mx : kOff;
#pragma unroll
  for (int t = 0; t < DT; ++t) out.acc[t] = acc[t];
}

template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_fwd4_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int S, int H, float sc,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ merged, int64_t ldm,
                                                         float* __restrict__ ml) {
  constexpr int W = HD / 4;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, D = H * HD, items = N * H;
  const size_t bufsz = KV<HD>::floats(NW);
  const int l = threadIdx.x & 63, g = l >> 4, i = 16 * (threadIdx.x >> 6) + (l & 15);
  int item = blockIdx.x;
  if (item >= items) return;
  Atom at(off, item, H, N, S);
  float pq[W];
  auto fetch_q = [&](const Atom& a) {
    if (i < a.cnt)
      gmem_get<W>(qkv + a.row(i) * ldq + a.h * HD + g * W, pq);
    else
#pragma unroll
      for (int t = 0; t < W; ++t) pq[t] = 0.f;
  };
  int buf = 0;
  kv_issue<HD>(lds, qkv, ldq, D, cf_seq, ldc, at);
  fetch_q(at);
  FwdOut<HD> out;
  Atom done = at;
  bool pending = false;
  for (;;) {
    wait_vm_all();
    lds_barrier();
    float q[W];
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = pq[t];
    const Atom cur = at;
    const float* cb = lds + buf * bufsz;
    const int next = item + gridDim.x;
    if (next < items) {
      at = Atom(off, next, H, N, S);
      kv_issue<HD>(lds + (buf ^ 1) * bufsz, qkv, ldq, D, cf_seq, ldc, at);
      fetch_q(at);
    }
    if (pending) fwd_store<HD>(done, out, S, H, merged, ldm, ml);
    fwd_item_kv<HD>(cur, cb, q, sc, out);
    done = cur;
    pending = true;
    buf ^= 1;
    if (next >= items) break;
    item = next;
  }
  fwd_store<HD>(done, out, S, H, merged, ldm, ml);
}

// ---- backward --------------------------------------------------------------
// A lane's share of one item's backward result, held until it is stored.
template <int HD>
struct BwdOut {
  f4 dq[HD / 16], dk[HD / 16], dv[HD / 16];
  float cft;
};

// One item's backward from the staged Q, K, dO (and V) and log cf.
template <int HD>
__device__ __forceinline__ void bwd_item(const Atom& at, const float* Qs, const float* Ks, const float* Gs,
                                         const float* Vs, const float* lcf, float* Tb, int nbuf, int vlds,
                                         const float* oo, float mi, float li, const float* __restrict__ qkv,
                                         int64_t ldq, int H, float sc, BwdOut<HD>& out) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P, TP = Lds<HD>::TP, TILE = 16 * TP;
  const int NW = blockDim.x >> 6, D = H * HD;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bool active = w < at.nb;
  const int i = 16 * w + c;  // this lane's query slot, and its key slot
  float q[W], go[W], dqi = 0.f;
  if (active) {
    lds_get<W>(Qs + i * P + g * W, q);
    lds_get<W>(Gs + i * P + g * W, go);
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < W; ++t) d += go[t] * oo[t];
    dqi = sum_g(d);  // Dq = dO . O of query i
  }
  f4 dq[DT], dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  const int nb = at.nb;
  // Phase 1 of step s: tile (query block w, key block J = (w + s) mod nb):
  // S^T and dP^T, then A and dS, the dQ share, and A, dS left in LDS.
  auto phase1 = [&](int s, bool v_staged) {
    float* tb = Tb + (nbuf == 2 ? (s & 1) : 0) * (NW * 2 * TILE);
    int J = w + s;
    if (J >= nb) J -= nb;
    f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
    {
      float k[W], v[W];
      lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
      if (v_staged)
        lds_get<W>(Vs + (16 * J + c) * P + g * W, v);
      else if (16 * J + c < at.cnt)
        gmem_get<W>(qkv + at.row(16 * J + c) * ldq + 2 * D + at.h * HD + g * W, v);
      else
#pragma unroll
        for (int t = 0; t < W; ++t) v[t] = 0.f;
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
  };
  // Phase 2 of step s: key block w's tile from query block Ip = (w - s) mod nb:
  // dK^T += Q^T dS, dV^T += dO^T A, and the key's dS summed.
  auto phase2 = [&](int s) {
    const float* tb = Tb + (nbuf == 2 ? (s & 1) : 0) * (NW * 2 * TILE);
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
  };
  if (nbuf == 2 && vlds) {
    // Software-pipelined: between two barriers a wave has phase 2 of the last
    // step and phase 1 of this one, independent work the scheduler interleaves.
    if (active) phase1(0, true);
    lds_barrier();
    for (int s = 1; s < nb; ++s) {
      if (active) {
        phase2(s - 1);
        phase1(s, true);
      }
      lds_barrier();
    }
    if (active) phase2(nb - 1);
  } else {
    for (int s = 0; s < nb; ++s) {
      if (active) phase1(s, vlds != 0);
      lds_barrier();
      if (active) phase2(s);
      if (nbuf == 1) lds_barrier();  // the owners are done with the only buffer
    }
  }
  out.cft = sum_g(cfa);
#pragma unroll
  for (int t = 0; t < DT; ++t) out.dq[t] = dq[t], out.dk[t] = dk[t], out.dv[t] = dv[t];
}

// The item's stores: dQ | dK | dV rows of its tokens, its row of cfh.
template <int HD>
__device__ __forceinline__ void bwd_store(const Atom& at, const BwdOut<HD>& out, int S, int H, float sc,
                                          float* __restrict__ qkv_adj, int64_t lda, float* __restrict__ cfh) {
  constexpr int W = HD / 4;
  const int D = H * HD;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;
  const bool real = w < at.nb && i < at.cnt;
  if (real) {
    float* o = qkv_adj + at.row(i) * lda + at.h * HD + g * W;
    store_slice<HD>(o, out.dq, sc);
    store_slice<HD>(o + D, out.dk, sc);
    store_slice<HD>(o + 2 * D, out.dv, 1.0f);
  }
  // cfh [N][H][S]: one contiguous row of S per item
  if (g == 0 && i < S) cfh[(size_t(at.n) * H + at.h) * S + i] = real ? out.cft : 0.f;
}

template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_bwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int S, int H, float sc,
                                                        const float* __restrict__ dmerged, int64_t ldg,
                                                        const float* __restrict__ merged, int64_t ldm,
                                                        const float* __restrict__ ml,
                                                        const float* __restrict__ cf_seq, int64_t ldc,
                                                        float* __restrict__ qkv_adj, int64_t lda,
                                                        float* __restrict__ cfh, int nbuf, int vlds) {
  constexpr int W = HD / 4, P = Lds<HD>::P;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD, items = N * H;
  float* Qs = lds;
  float* Ks = Qs + R * P;
  float* Gs = Ks + R * P;
  float* Vs = Gs + R * P;  // when vlds
  float* lcf = Vs + (vlds ? R * P : 0);
  float* Tb = lcf + R;  // [nbuf buffers][NW producers][A, dS][16 x TP]
  const int l = threadIdx.x & 63, g = l >> 4, i = 16 * (threadIdx.x >> 6) + (l & 15);
  int item = blockIdx.x;
  if (item >= items) return;
  Atom at(off, item, H, N, S);
  SliceRegs<HD> pq, pk, pg, pv;
  float pcf, poo[W], pm, pl;
  auto fetch = [&](const Atom& a) {
    pq.load(qkv, ldq, a.h * HD, a);
    pk.load(qkv, ldq, D + a.h * HD, a);
    pg.load(dmerged, ldg, a.h * HD, a);
    if (vlds) pv.load(qkv, ldq, 2 * D + a.h * HD, a);
    pcf = int(threadIdx.x) < a.cnt ? cf_seq[size_t(a.n) * ldc + threadIdx.x] : 0.f;
    pm = kOff, pl = 0.f;
    if (i < a.cnt) {
      gmem_get<W>(merged + a.row(i) * ldm + a.h * HD + g * W, poo);
      const float* m2 = ml + 2 * ((size_t(a.n) * H + a.h) * S + i);
      pm = m2[0], pl = m2[1];
    } else {
#pragma unroll
      for (int t = 0; t < W; ++t) poo[t] = 0.f;
    }
  };
  fetch(at);
  BwdOut<HD> out;
  Atom done = at;
  bool pending = false;
  for (;;) {
    pq.template store<P>(Qs);
    pk.template store<P>(Ks);
    pg.template store<P>(Gs);
    if (vlds) pv.template store<P>(Vs);
    if (int(threadIdx.x) < R) lcf[threadIdx.x] = pcf > 0.f ? __logf(pcf) : kOff;
    float oo[W];
#pragma unroll
    for (int t = 0; t < W; ++t) oo[t] = poo[t];
    const float mi = pm, li = pl;
    if (pending) bwd_store<HD>(done, out, S, H, sc, qkv_adj, lda, cfh);
    const Atom cur = at;
    lds_barrier();
    const int next = item + gridDim.x;
    if (next < items) {
      at = Atom(off, next, H, N, S);
      fetch(at);
    }
    bwd_item<HD>(cur, Qs, Ks, Gs, Vs, lcf, Tb, nbuf, vlds, oo, mi, li, qkv, ldq, H, sc, out);
    done = cur;
    pending = true;
    if (next >= items) break;
    lds_barrier();
    item = next;
  }
  bwd_store<HD>(done, out, S, H, sc, qkv_adj, lda, cfh);
}

// One item per workgroup: the item's slices, its own rows' O and statistics
// loaded into registers, staged in LDS, one barrier, then its backward.
template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_bwd1_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int S, int H, float sc,
                                                         const float* __restrict__ dmerged, int64_t ldg,
                                                         const float* __restrict__ merged, int64_t ldm,
                                                         const float* __restrict__ ml,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ qkv_adj, int64_t lda,
                                                         float* __restrict__ cfh, int nbuf, int vlds) {
  constexpr int W = HD / 4, P = Lds<HD>::P;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD;
  float* Qs = lds;
  float* Ks = Qs + R * P;
  float* Gs = Ks + R * P;
  float* Vs = Gs + R * P;  // when vlds
  float* lcf = Vs + (vlds ? R * P : 0);
  float* Tb = lcf + R;
  const int l = threadIdx.x & 63, g = l >> 4, i = 16 * (threadIdx.x >> 6) + (l & 15);
  const Atom at(off, blockIdx.x, H, N, S);
  float oo[W], mi = kOff, li = 0.f;
  {
    SliceRegs<HD> pq, pk, pg, pv;
    pq.load(qkv, ldq, at.h * HD, at);
    pk.load(qkv, ldq, D + at.h * HD, at);
    pg.load(dmerged, ldg, at.h * HD, at);
    if (vlds) pv.load(qkv, ldq, 2 * D + at.h * HD, at);
    const float pcf = int(threadIdx.x) < at.cnt ? cf_seq[size_t(at.n) * ldc + threadIdx.x] : 0.f;
    if (i < at.cnt) {
      gmem_get<W>(merged + at.row(i) * ldm + at.h * HD + g * W, oo);
      const float* m2 = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
      mi = m2[0], li = m2[1];
    } else {
#pragma unroll
      for (int t = 0; t < W; ++t) oo[t] = 0.f;
    }
    pq.template store<P>(Qs);
    pk.template store<P>(Ks);
    pg.template store<P>(Gs);
    if (vlds) pv.template store<P>(Vs);
    if (int(threadIdx.x) < R) lcf[threadIdx.x] = pcf > 0.f ? __logf(pcf) : kOff;
  }
  lds_barrier();
  BwdOut<HD> out;
  bwd_item<HD>(at, Qs, Ks, Gs, Vs, lcf, Tb, nbuf, vlds, oo, mi, li, qkv, ldq, H, sc, out);
  bwd_store<HD>(at, out, S, H, sc, qkv_adj, lda, cfh);
}

// ---- backward v2: 3 workgroups a CU ---------------------------------------------
// Q, K and dO staged at pitch hd (no padding): float4 q of row r sits at
// q ^ key(r), key(r) = r & 7 when a row covers the 32 banks (hd a multiple of
// 32), (r >> 1) & 3 at hd 16 (two rows per 32 banks). Eight consecutive rows
// read at one float4 column (the MFMA row operands) and one row read across
// its columns (the transposed operands) then touch distinct banks.
template <int HD>
struct SwSlice {
  static constexpr int C4 = HD / 4;
  __device__ static __forceinline__ int key(int r) { return HD == 16 ? (r >> 1) & 3 : r & 7; }
  __device__ static __forceinline__ int f4(int r, int q) { return r * C4 + (q ^ key(r)); }
  __device__ static __forceinline__ int fl(int r, int x) { return 4 * f4(r, x >> 2) + (x & 3); }
};
// A 16 x 16 tile at pitch 16: row r stored as row r ^ ((r >> 2) & 1), its
// float4 q at q ^ ((stored row >> 1) & 3). The producer's 128-bit row writes
// (eight rows a pass) and the consumer's 32-bit column reads (rows 4g + r of
// two g a pass) are then both free of bank conflicts.
struct SwTile {
  __device__ static __forceinline__ int prow(int r) { return r ^ ((r >> 2) & 1); }
  __device__ static __forceinline__ int f4(int r, int q) {
    const int p = prow(r);
    return 4 * p + (q ^ ((p >> 1) & 3));
  }
  __device__ static __forceinline__ int fl(int r, int x) { return 4 * f4(r, x >> 2) + (x & 3); }
};

// DT consecutive floats x0 .. x0 + DT - 1 (x0 a multiple of DT) of row r.
template <int HD, int DT>
__device__ __forceinline__ void sw_get(const float* base, int r, int x0, float* out) {
  if constexpr (DT % 4 == 0) {
#pragma unroll
    for (int j = 0; j < DT; j += 4) {
      const float4 v = *reinterpret_cast<const float4*>(base + 4 * SwSlice<HD>::f4(r, (x0 + j) >> 2));
      out[j] = v.x, out[j + 1] = v.y, out[j + 2] = v.z, out[j + 3] = v.w;
    }
  } else if constexpr (DT % 2 == 0) {
#pragma unroll
    for (int j = 0; j < DT; j += 2) {
      const float2 v = *reinterpret_cast<const float2*>(base + SwSlice<HD>::fl(r, x0 + j));
      out[j] = v.x, out[j + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < DT; ++j) out[j] = base[SwSlice<HD>::fl(r, x0 + j)];
  }
}

template <int HD>
struct LdsV2 {
  // Q, K, dO at pitch hd, log cf, two buffers of [NW producers][A, dS] tiles.
  static size_t floats(int NW) { return size_t(3) * NW * 16 * HD + NW * 16 + size_t(2) * NW * 2 * 256; }
};

template <int HD, int MAXT>
__global__ void __launch_bounds__(MAXT) attn_bwd2_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int S, int H, float sc,
                                                         const float* __restrict__ dmerged, int64_t ldg,
                                                         const float* __restrict__ merged, int64_t ldm,
                                                         const float* __restrict__ ml,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ qkv_adj, int64_t lda,
                                                         float* __restrict__ cfh) {
  constexpr int W = HD / 4, DT = HD / 16, C4 = HD / 4;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD;
  float* Qs = lds;
  float* Ks = Qs + R * HD;
  float* Gs = Ks + R * HD;
  float* lcf = Gs + R * HD;
  float* Tb = lcf + R;  // [2][NW][A, dS][256]
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;
  const Atom at(off, blockIdx.x, H, N, S);
  const int nb = at.nb;
  const bool active = w < nb;
  const float* Vg = qkv + 2 * D + at.h * HD;
  // V row 16J + c, this lane's slice. A row past the count loads the atom's
  // own row instead: finite values for a key whose weight is zero, and no
  // select on the loaded registers, which would wait for the load.
  auto load_v = [&](int J, float* v) {
    const int r = 16 * J + c;
    gmem_get<W>(Vg + at.row(r < at.cnt ? r : 0) * ldq + g * W, v);
  };
  float oo[W], vcur[W], mi = kOff, li = 0.f;
  {
    SliceRegs<HD> pq, pk, pg;
    pq.load(qkv, ldq, at.h * HD, at);
    pk.load(qkv, ldq, D + at.h * HD, at);
    pg.load(dmerged, ldg, at.h * HD, at);
    const float pcf = int(threadIdx.x) < at.cnt ? cf_seq[size_t(at.n) * ldc + threadIdx.x] : 0.f;
    if (i < at.cnt) {
      gmem_get<W>(merged + at.row(i) * ldm + at.h * HD + g * W, oo);
      const float* m2 = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
      mi = m2[0], li = m2[1];
    } else {
#pragma unroll
      for (int t = 0; t < W; ++t) oo[t] = 0.f;
    }
    if (active) load_v(w, vcur);  // step 0's key block is w
#pragma unroll
    for (int k = 0; k < SliceRegs<HD>::PER; ++k) {
      const int idx = threadIdx.x + k * blockDim.x, r = idx / C4, q = idx - r * C4;
      const int o = 4 * SwSlice<HD>::f4(r, q);
      *reinterpret_cast<float4*>(Qs + o) = pq.v[k];
      *reinterpret_cast<float4*>(Ks + o) = pk.v[k];
      *reinterpret_cast<float4*>(Gs + o) = pg.v[k];
    }
    if (int(threadIdx.x) < R) lcf[threadIdx.x] = pcf > 0.f ? __logf(pcf) : kOff;
  }
  lds_barrier();

  float q[W], go[W], dqi = 0.f;
  if (active) {
#pragma unroll
    for (int u = 0; u < W / 4; ++u) {
      const float4 a = *reinterpret_cast<const float4*>(Qs + 4 * SwSlice<HD>::f4(i, g * (W / 4) + u));
      const float4 b = *reinterpret_cast<const float4*>(Gs + 4 * SwSlice<HD>::f4(i, g * (W / 4) + u));
      q[4 * u] = a.x, q[4 * u + 1] = a.y, q[4 * u + 2] = a.z, q[4 * u + 3] = a.w;
      go[4 * u] = b.x, go[4 * u + 1] = b.y, go[4 * u + 2] = b.z, go[4 * u + 3] = b.w;
    }
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < W; ++t) d += go[t] * oo[t];
    dqi = sum_g(d);  // Dq = dO . O of query i
  }
  f4 dq[DT], dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  auto phase1 = [&](int s, const float* v) {
    float* ta = Tb + ((s & 1) * NW + w) * 512;
    int J = w + s;
    if (J >= nb) J -= nb;
    f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
    {
      const int rk = 16 * J + c;
      float k[W];
#pragma unroll
      for (int u = 0; u < W / 4; ++u) {
        const float4 a = *reinterpret_cast<const float4*>(Ks + 4 * SwSlice<HD>::f4(rk, g * (W / 4) + u));
        k[4 * u] = a.x, k[4 * u + 1] = a.y, k[4 * u + 2] = a.z, k[4 * u + 3] = a.w;
      }
#pragma unroll
      for (int t = 0; t < W; ++t) st = mfma(k[t], q[t], st), dp = mfma(v[t], go[t], dp);
    }
    float lc[4], a[4], ds[4];
    lds_get<4>(lcf + 16 * J + 4 * g, lc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      a[r] = li > 0.f && !is_off(lc[r]) ? __expf(st[r] * sc + lc[r] - mi) * li : 0.f;
      ds[r] = a[r] * (dp[r] - dqi);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float kk[DT];
      sw_get<HD, DT>(Ks, 16 * J + 4 * g + r, c * DT, kk);
#pragma unroll
      for (int t = 0; t < DT; ++t) dq[t] = mfma(kk[t], ds[r], dq[t]);
    }
    *reinterpret_cast<float4*>(ta + 4 * SwTile::f4(c, g)) = make_float4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<float4*>(ta + 256 + 4 * SwTile::f4(c, g)) = make_float4(ds[0], ds[1], ds[2], ds[3]);
  };
  auto phase2 = [&](int s) {
    int Ip = w - s;
    if (Ip < 0) Ip += nb;
    const float* ta = Tb + ((s & 1) * NW + Ip) * 512;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = SwTile::fl(4 * g + r, c);
      const float av = ta[o], dsv = ta[256 + o];
      cfa += dsv;
      float qq[DT], gg[DT];
      sw_get<HD, DT>(Qs, 16 * Ip + 4 * g + r, c * DT, qq);
      sw_get<HD, DT>(Gs, 16 * Ip + 4 * g + r, c * DT, gg);
#pragma unroll
      for (int t = 0; t < DT; ++t) dk[t] = mfma(qq[t], dsv, dk[t]), dv[t] = mfma(gg[t], av, dv[t]);
    }
  };
  // Pipelined steps: between two barriers a wave has phase 2 of the last step,
  // phase 1 of this one and the V rows of the next in flight. The V rows
  // alternate between two register sets (steps taken two at a time), so a
  // load is first used a whole step after it is issued.
  float valt[W];
  auto key_block = [&](int s) {
    int J = w + s;
    while (J >= nb) J -= nb;
    return J;
  };
  if (active) {
    load_v(key_block(1), valt);
    phase1(0, vcur);
  }
  lds_barrier();
  for (int s = 1; s < nb; s += 2) {
    if (active) {
      load_v(key_block(s + 1), vcur);  // step s + 1's rows, into the set step s - 1 used
      phase2(s - 1);
      phase1(s, valt);
    }
    lds_barrier();
    if (s + 1 < nb) {
      if (active) {
        load_v(key_block(s + 2), valt);
        phase2(s);
        phase1(s + 1, vcur);
      }
      lds_barrier();
    }
  }
  if (active) phase2(nb - 1);
  BwdOut<HD> out;
  out.cft = sum_g(cfa);
#pragma unroll
  for (int t = 0; t < DT; ++t) out.dq[t] = dq[t], out.dk[t] = dk[t], out.dv[t] = dv[t];
  bwd_store<HD>(at, out, S, H, sc, qkv_adj, lda, cfh);
}

// cf_seq_adj(n, k) += sum_h cfh[n][h][k] / cf(n, k) where cf > 0, heads in
// order (the reference's attn_bwd_cf, src/attention.cpp:1829-1838).
__global__ void attn_cf_adjoint_kernel(const float* __restrict__ cfh, const float* __restrict__ cf_seq, int64_t ldc,
                                       float* __restrict__ cf_seq_adj, int64_t ldca, int N, int S, int H) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(N) * S) return;
  const int n = int(i / S), k = int(i - int64_t(n) * S);
  const float cf = cf_seq[int64_t(n) * ldc + k];
  if (cf <= 0.f) return;
  float total = 0.f;
  for (int hh = 0; hh < H; ++hh) total += cfh[(int64_t(n) * H + hh) * S + k];
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

// Tuning knobs read once from the environment (0 or unset: automatic).
int env_int(const char* name) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : 0;
}

// The persistent grid: workgroups resident at once for kernel k at this block
// size and LDS, times the device's CUs (times PET_ATTN_GRID_MULT), never more
// than the items. Cached per (kernel, device, block, bytes).
unsigned persistent_grid(const void* k, int block, size_t bytes, int64_t items) {
  struct Key {
    const void* k;
    int dev, block;
    size_t bytes;
  };
  static std::mutex mu;
  static std::vector<std::pair<Key, int64_t>> cache;
  int dev = 0;
  (void) hipGetDevice(&dev);
  int64_t per = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (auto& e : cache)
      if (e.first.k == k && e.first.dev == dev && e.first.block == block && e.first.bytes == bytes) per = e.second;
    if (per == 0) {
      int cus = 0, occ = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, block, bytes) != hipSuccess || occ < 1) occ = 1;
      static const int mult = env_int("PET_ATTN_GRID_MULT");
      per = int64_t(cus) * occ * (mult > 0 ? mult : 1);
      cache.push_back({Key{k, dev, block, bytes}, per});
    }
  }
  return unsigned(per < items ? per : items);
}

template <class K>
void allow_lds(K k, size_t bytes) {
  if (bytes > 65536)
    (void) hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(bytes));
}

template <int HD>
int launch_fwd(const pet_attn_shape& sh, const float* qkv, int64_t ldq, const int* off, const float* cf_seq,
               int64_t ldc, float* merged, int64_t ldm, float* ml, hipStream_t st) {
  const int NW = waves_for(sh.slots);
  const size_t bytes = sizeof(float) * Lds<HD>::fwd_floats(NW);
  if (bytes > size_t(max_lds_bytes())) return PET_ATTN_ESLOTS;
  const int64_t items = int64_t(sh.n_atoms) * sh.heads;
  const int block = 64 * NW;
  static const int variant = env_int("PET_ATTN_FWD_VARIANT") ? env_int("PET_ATTN_FWD_VARIANT") : 1;
  const size_t b4 = 2 * sizeof(float) * KV<HD>::floats(NW);
  if (variant == 4 && b4 <= size_t(max_lds_bytes())) {
    auto k4 = NW <= 8 ? attn_fwd4_kernel<HD, 512> : attn_fwd4_kernel<HD, 1024>;
    allow_lds(k4, b4);
    const unsigned grid = persistent_grid(reinterpret_cast<const void*>(k4), block, b4, items);
    hipLaunchKernelGGL(k4, dim3(grid), dim3(block), b4, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads,
                       sh.scale, cf_seq, ldc, merged, ldm, ml);
    return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
  }
  if (variant == 1 || variant == 2 || variant == 4) {
    auto k1 = variant != 2 ? (NW <= 8 ? attn_fwd1_kernel<HD, 512> : attn_fwd1_kernel<HD, 1024>)
                           : (NW <= 8 ? attn_fwd2_kernel<HD, 512> : attn_fwd2_kernel<HD, 1024>);
    const size_t b1 = variant != 2 ? bytes : 0;
    allow_lds(k1, b1);
    hipLaunchKernelGGL(k1, dim3(unsigned(items)), dim3(block), b1, st, qkv, ldq, off, sh.n_atoms, sh.slots,
                       sh.heads, sh.scale, cf_seq, ldc, merged, ldm, ml);
    return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
  }
  auto k = variant == 3 ? (NW <= 8 ? attn_fwd3_kernel<HD, 512> : attn_fwd3_kernel<HD, 1024>)  // 9: persistent
                        : (NW <= 8 ? attn_fwd_kernel<HD, 512> : attn_fwd_kernel<HD, 1024>);
  allow_lds(k, bytes);
  const unsigned grid = persistent_grid(reinterpret_cast<const void*>(k), block, bytes, items);
  hipLaunchKernelGGL(k, dim3(grid), dim3(block), bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                     cf_seq, ldc, merged, ldm, ml);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

template <int HD>
int launch_bwd(const pet_attn_shape& sh, const float* qkv, int64_t ldq, const int* off, const float* dmerged,
               int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
               float* qkv_adj, int64_t lda, float* cfh, hipStream_t st) {
  const int NW = waves_for(sh.slots);
  // The fullest layout that fits: V staged and two tile buffers, else V from
  // global memory, else also one tile buffer. PET_ATTN_BWD_VLDS (1 staged,
  // 2 not) and PET_ATTN_BWD_NBUF (1, 2) force one where it fits.
  static const int force_v = env_int("PET_ATTN_BWD_VLDS"), force_b = env_int("PET_ATTN_BWD_NBUF");
  const size_t cap = size_t(max_lds_bytes());
  int nbuf = 2, vlds = 1;
  size_t bytes = sizeof(float) * Lds<HD>::bwd_floats(NW, nbuf, vlds);
  if (bytes > cap) vlds = 0, bytes = sizeof(float) * Lds<HD>::bwd_floats(NW, nbuf, vlds);
  if (bytes > cap) nbuf = 1, bytes = sizeof(float) * Lds<HD>::bwd_floats(NW, nbuf, vlds);
  if (bytes > cap) return PET_ATTN_ESLOTS;
  if (force_v || force_b) {
    const int v = force_v ? (force_v == 1) : vlds, b = force_b ? force_b : nbuf;
    const size_t fb = sizeof(float) * Lds<HD>::bwd_floats(NW, b, v);
    if ((b == 1 || b == 2) && fb <= cap) vlds = v, nbuf = b, bytes = fb;
  }
  const int64_t items = int64_t(sh.n_atoms) * sh.heads;
  const int block = 64 * NW;
  static const int variant = env_int("PET_ATTN_BWD_VARIANT");
  constexpr bool v2_layout = HD == 16 || HD % 32 == 0;
  const size_t b2 = sizeof(float) * LdsV2<HD>::floats(NW);
  if constexpr (v2_layout) {
    if (variant == 2 && b2 <= cap) {
      auto k2 = NW <= 8 ? attn_bwd2_kernel<HD, 512> : attn_bwd2_kernel<HD, 1024>;
      allow_lds(k2, b2);
      hipLaunchKernelGGL(k2, dim3(unsigned(items)), dim3(block), b2, st, qkv, ldq, off, sh.n_atoms, sh.slots,
                         sh.heads, sh.scale, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh);
      return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
    }
  }
  if (variant != 9) {  // one item per workgroup, padded layout
    auto k1 = NW <= 8 ? attn_bwd1_kernel<HD, 512> : attn_bwd1_kernel<HD, 1024>;
    allow_lds(k1, bytes);
    hipLaunchKernelGGL(k1, dim3(unsigned(items)), dim3(block), bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots,
                       sh.heads, sh.scale, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, nbuf, vlds);
    return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
  }
  auto k = NW <= 8 ? attn_bwd_kernel<HD, 512> : attn_bwd_kernel<HD, 1024>;
  allow_lds(k, bytes);
  const unsigned grid = persistent_grid(reinterpret_cast<const void*>(k), block, bytes, items);
  hipLaunchKernelGGL(k, dim3(grid), dim3(block), bytes, st, qkv, ldq, off, sh.n_atoms, sh.slots, sh.heads, sh.scale,
                     dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, nbuf, vlds);
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

int pet_attn_max_slots(int head_dim) {
  int e = with_head_dim(head_dim, [&](auto hd) {
    constexpr int HD = decltype(hd)::value;
    const size_t cap = size_t(max_lds_bytes());
    for (int NW = PET_ATTN_MAX_SLOTS / 16; NW >= 1; --NW)
      if (sizeof(float) * Lds<HD>::fwd_floats(NW) <= cap && sizeof(float) * Lds<HD>::bwd_floats(NW, 1, false) <= cap)
        return -16 * NW;  // negative: a count, not an error code
    return 0;
  });
  return e < 0 ? -e : 0;
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
