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

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/pet_attn.h"
#include "attn_common.h"
#include "split_bf16.h"

namespace pet_attn {

// ---- fp32 products on the bf16 matrix cores (split_bf16.h) -------------------
using pet_split::bf8;
using pet_split::mfma6;
using pet_split::mfma_bf;
using pet_split::pack_hi;
using pet_split::split3;
using pet_split::split8;
using pet_split::u4;

template <int HD>
struct Lds {
  static constexpr int P = HD + 4;   // row pitch of staged slices
  static constexpr int TP = 16 + 4;  // row pitch of a 16 x 16 tile
  // split K rows (forward scores on the bf16 matrix cores): per 8-dim group
  // its three parts, 8 bf16 each, then a 16-byte pad (rows 16-lane
  // conflict-free); in 4-byte words
  static constexpr int KP6 = 3 * HD / 2 + 4;
  static size_t fwd_floats(int NW, bool spl = false) {
    return size_t(spl ? KP6 + P : 2 * P) * NW * 16 + NW * 16;
  }
  // nbuf tile buffers: 2 lets a step's producers write while the last step's
  // owners still read (one barrier a step); 1 needs two barriers a step.
  // vlds: V staged too (else its rows come from global memory).
  // spl: V staged as split rows (pitch KP6) for dP^T on the bf16 matrix cores
  static size_t bwd_floats(int NW, int nbuf, bool vlds, bool spl = false) {
    return (size_t(3) * P + (vlds ? (spl ? KP6 : P) : 0)) * NW * 16 + NW * 16 + size_t(nbuf) * NW * 2 * 16 * TP;
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
template <int HD, bool SPL>
__device__ __forceinline__ void fwd_item(const Atom& at, const float* Ks, const float* Vs, const float* lcf,
                                         const float* q, const u4* qs, float sc, FwdOut<HD>& out) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P, KP6 = Lds<HD>::KP6;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;  // this lane's query slot
  if (w >= at.nb) {  // slots past the atom's tokens: only the workgroup barrier
    lds_barrier();
    return;
  }
  float mx = kFloor, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  // S^T of key block J: s[r] = query i against key 16J + 4g + r.
  auto scores = [&](int J) {
    f4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (SPL) {
      const unsigned* kb = reinterpret_cast<const unsigned*>(Ks) + (16 * J + c) * KP6 + g * (W / 8) * 12;
#pragma unroll
      for (int kc = 0; kc < W / 8; ++kc) {
        u4 a[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) a[p] = *reinterpret_cast<const u4*>(kb + kc * 12 + 4 * p);
        s = mfma6(a, qs + 3 * kc, s);
      }
    } else {
      float k[W];
      lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
#pragma unroll
      for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);
    }
    return s;
  };
  // Online softmax and PV of key block J from its scores s.
  auto block = [&](int J, const f4& s) {
    float lc[4];
    lds_get<4>(lcf + 16 * J + 4 * g, lc);
    float x[4], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s[r] * sc + lc[r];
      bm = fmaxf(bm, x[r]);
    }
    const float nm = fmaxf(mx, max_g(bm));
    const float alpha = __expf(mx - nm);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __expf(x[r] - nm);
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
  // Two key blocks at a time: one max, one rescale of acc and sum for 32
  // keys instead of 16.
  auto block2 = [&](int J0, const f4& s0, int J1, const f4& s1) {
    float lc[8];
    lds_get<4>(lcf + 16 * J0 + 4 * g, lc);
    lds_get<4>(lcf + 16 * J1 + 4 * g, lc + 4);
    float x[8], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = s0[r] * sc + lc[r];
      x[4 + r] = s1[r] * sc + lc[4 + r];
      bm = fmaxf(bm, fmaxf(x[r], x[4 + r]));
    }
    const float nm = fmaxf(mx, max_g(bm));
    const float alpha = __expf(mx - nm);
    float p[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) p[r] = __expf(x[r] - nm);
    sum = sum * alpha + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
    mx = nm;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= alpha;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v[DT];
        lds_get<DT>(Vs + (16 * (h ? J1 : J0) + 4 * g + r) * P + c * DT, v);
#pragma unroll
        for (int t = 0; t < DT; ++t) acc[t] = mfma(v[t], p[4 * h + r], acc[t]);
      }
  };
  // The wave's own key block first: it is all the wave itself staged, so it
  // runs before the workgroup barrier, under the other waves' loads. Then the
  // others in the order w + 1, w + 2, ... (mod nb), two at a time (their two
  // score products independent), an odd one last.
  block(w, scores(w));
  lds_barrier();
  auto next = [&](int j) { return j + 1 < at.nb ? j + 1 : 0; };
  int rem = at.nb - 1, J0 = next(w);
  for (; rem >= 2; rem -= 2) {
    const int J1 = next(J0);
    const f4 s0 = scores(J0), s1 = scores(J1);
    block2(J0, s0, J1, s1);
    J0 = next(J1);
  }
  if (rem == 1) block(J0, scores(J0));
  const float tot = sum_g(sum);
  // else a query on an edge at its cutoff: zeros
  out.live = i < at.cnt && (i == 0 || !is_off(lcf[i]));
  out.invl = out.live && tot > 0.f ? 1.0f / tot : 0.f;
  out.mx = out.live && tot > 0.f ? mx : kOff;  // no live key: the max never left kFloor
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
  if (w < at.nb && i < at.cnt) store_slice<HD>(merged + at.grow(i) * ldm + at.h * HD + g * W, out.acc, out.invl);
  if (ml && g == 0) {
    float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    const bool real = w < at.nb && i < at.cnt;
    mlq[0] = real ? out.mx : kOff, mlq[1] = real ? out.invl : 0.f;
  }
}

// One item per workgroup: the item's K, V and q loaded into registers and
// staged in LDS, one barrier, then its forward.
template <int HD, int MAXT, bool XF = false, bool SPL = false>
// At head_dim <= 32 the forward is held to 64 VGPRs (eight waves a SIMD: five
// 5-wave workgroups a CU), which it fits without spilling.
__global__ void __launch_bounds__(MAXT) __attribute__((amdgpu_waves_per_eu(HD <= 32 ? 8 : 1))) attn_fwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int n0, int64_t eb,
                                                        int S, int H, float sc, const float* __restrict__ cf_seq,
                                                        int64_t ldc, float* __restrict__ merged, int64_t ldm,
                                                        float* __restrict__ ml, QkvXf xf) {
  static_assert(!SPL || HD % 32 == 0, "split scores take 32-dim products");
  constexpr int W = HD / 4, P = Lds<HD>::P, KP6 = Lds<HD>::KP6;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD;
  float* Ks = lds;
  float* Vs = Ks + R * (SPL ? KP6 : P);
  float* lcf = Vs + R * P;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, i = 16 * w + (l & 15);
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, n0, eb);
  // Each wave stages its own block -- rows 16w .. 16w+15 of K and V, lane
  // (c, g) the slice of row 16w + c it also loads q from -- and its keys' cf;
  // the workgroup barrier is inside fwd_item, after the wave's own block.
  float q[W];
  u4 qs[SPL ? 3 * (W / 8) : 1];
  if (w < at.nb) {
    float k[W], v[W];
    const bool real = i < at.cnt;
    // A padded slot (i >= cnt) loads the atom's own row instead of zeros: its
    // values are finite (and cached), its key's log cf is kOff so its weight
    // is exactly 0, and its query's results are not stored; no branch.
    const size_t r = at.row(real ? i : 0);
    qkv_get<W, XF>(qkv, ldq, r, at.h * HD + g * W, xf, q);
    qkv_get<W, XF>(qkv, ldq, r, D + at.h * HD + g * W, xf, k);
    qkv_get<W, XF>(qkv, ldq, r, 2 * D + at.h * HD + g * W, xf, v);
    const float pcf = real && g == 0 ? cf_seq[size_t(at.n) * ldc + i] : 0.f;
    if constexpr (SPL) {
      unsigned* o = reinterpret_cast<unsigned*>(Ks) + i * KP6 + g * (W / 8) * 12;
#pragma unroll
      for (int kc = 0; kc < W / 8; ++kc) {
        u4 kp[3];
        split8(k + 8 * kc, kp);
        split8(q + 8 * kc, qs + 3 * kc);
#pragma unroll
        for (int p = 0; p < 3; ++p) *reinterpret_cast<u4*>(o + kc * 12 + 4 * p) = kp[p];
      }
    }
    float* ok = Ks + i * P + g * W;  // fp32 K rows (unsplit)
    float* ov = Vs + i * P + g * W;
#pragma unroll
    for (int t = 0; t < W; t += 4) {
      if constexpr (!SPL) *reinterpret_cast<float4*>(ok + t) = make_float4(k[t], k[t + 1], k[t + 2], k[t + 3]);
      *reinterpret_cast<float4*>(ov + t) = make_float4(v[t], v[t + 1], v[t + 2], v[t + 3]);
    }
    if (g == 0) lcf[i] = pcf > 0.f ? log_cf(pcf) : kOff;
  }
  FwdOut<HD> out;
  fwd_item<HD, SPL>(at, Ks, Vs, lcf, q, qs, sc, out);
  fwd_store<HD>(at, out, S, H, merged, ldm, ml);
}

// ---- forward on the vector ALUs (for comparison) ----------------------------
// The same forward with no matrix cores: a thread per query slot, the item's K
// and V rows staged in LDS and read by every lane at once (broadcast), online
// softmax over the keys four at a time. No padding to 16-token blocks, but each
// score and each weighted V row is hd fp32 FMAs on the vector ALUs (a wave64
// instruction every 4 cycles) instead of a quarter of a matrix-core product.
// Selected by option PET_OPT_FWD_KERNEL 3 (head_dim <= 64); the matrix-core kernel is the
// default.
template <int HD>
__global__ void __launch_bounds__(256) attn_fwd_valu_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                            const int* __restrict__ off, int N, int n0, int64_t eb,
                                                            int S, int H, float sc, const float* __restrict__ cf_seq,
                                                            int64_t ldc, float* __restrict__ merged, int64_t ldm,
                                                            float* __restrict__ ml) {
  constexpr int C4 = HD / 4;
  extern __shared__ float lds[];
  const int D = H * HD, R = blockDim.x;
  float* Ks = lds;
  float* Vs = Ks + R * HD;
  float* lcf = Vs + R * HD;
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, n0, eb);
  for (int f = threadIdx.x; f < at.cnt * C4; f += blockDim.x) {
    const int r = f / C4, c4 = f - r * C4;
    const float* src = qkv + at.row(r) * ldq + at.h * HD + 4 * c4;
    *reinterpret_cast<float4*>(Ks + r * HD + 4 * c4) = *reinterpret_cast<const float4*>(src + D);
    *reinterpret_cast<float4*>(Vs + r * HD + 4 * c4) = *reinterpret_cast<const float4*>(src + 2 * D);
  }
  const int i = threadIdx.x;
  if (i < at.cnt) {
    const float cv = cf_seq[size_t(at.n) * ldc + i];
    lcf[i] = cv > 0.f ? log_cf(cv) : kOff;
  }
  float q[HD], acc[HD];
  if (i < at.cnt) gmem_get<HD>(qkv + at.row(i) * ldq + at.h * HD, q);
  __syncthreads();
  if (i >= S) return;
  float mx = kOff, sum = 0.f;
#pragma unroll
  for (int t = 0; t < HD; ++t) acc[t] = 0.f;
  if (i < at.cnt) {
    for (int k0 = 0; k0 < at.cnt; k0 += 4) {
      float x[4], bm = kOff;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int k = k0 + u;
        const float lc = k < at.cnt ? lcf[k] : kOff;
        float d = 0.f;
        if (!is_off(lc)) {
#pragma unroll
          for (int t = 0; t < HD; t += 4) {
            const float4 kk = *reinterpret_cast<const float4*>(Ks + k * HD + t);
            d = fmaf(q[t], kk.x, d), d = fmaf(q[t + 1], kk.y, d), d = fmaf(q[t + 2], kk.z, d), d = fmaf(q[t + 3], kk.w, d);
          }
        }
        x[u] = is_off(lc) ? kOff : d * sc + lc;
        bm = fmaxf(bm, x[u]);
      }
      const float nm = fmaxf(mx, bm);
      const float alpha = __expf(mx - nm);
      float p[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) p[u] = is_off(x[u]) ? 0.f : __expf(x[u] - nm);
      sum = sum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      mx = nm;
#pragma unroll
      for (int t = 0; t < HD; ++t) acc[t] *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (p[u] == 0.f) continue;
        const int k = k0 + u;
#pragma unroll
        for (int t = 0; t < HD; t += 4) {
          const float4 vv = *reinterpret_cast<const float4*>(Vs + k * HD + t);
          acc[t] = fmaf(p[u], vv.x, acc[t]), acc[t + 1] = fmaf(p[u], vv.y, acc[t + 1]);
          acc[t + 2] = fmaf(p[u], vv.z, acc[t + 2]), acc[t + 3] = fmaf(p[u], vv.w, acc[t + 3]);
        }
      }
    }
  }
  const bool real = i < at.cnt;
  const bool live = real && (i == 0 || !is_off(lcf[i]));
  const float invl = live && sum > 0.f ? 1.0f / sum : 0.f;
  if (real) {
    float* o = merged + at.grow(i) * ldm + at.h * HD;
#pragma unroll
    for (int t = 0; t < HD; t += 4)
      *reinterpret_cast<float4*>(o + t) = make_float4(acc[t] * invl, acc[t + 1] * invl, acc[t + 2] * invl, acc[t + 3] * invl);
  }
  if (ml) {
    float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    mlq[0] = live ? mx : kOff, mlq[1] = invl;
  }
}

// ---- backward --------------------------------------------------------------
// a * b for small non-negative indices (a row index times a pitch): the
// full-rate 24-bit multiply instead of the quarter-rate 32-bit one.
__device__ __forceinline__ int mul24(int a, int b) { return int(__umul24(unsigned(a), unsigned(b))); }
// A lane's share of one item's backward result, held until it is stored.
template <int HD>
struct BwdOut {
  f4 dq[HD / 16], dk[HD / 16], dv[HD / 16];
  float cft;
};

// One item's backward from the staged Q, K, dO (and V) and log cf.
template <int HD, bool XF, bool SPL>
__device__ __forceinline__ void bwd_item(const Atom& at, const float* Qs, const float* Ks, const float* Gs,
                                         const float* Vs, const float* lcf, float* Tb, int nbuf, int vlds,
                                         const float* oo, float mi, float li, const float* __restrict__ qkv,
                                         int64_t ldq, const QkvXf& xf, int H, float sc, BwdOut<HD>& out) {
  constexpr int W = HD / 4, DT = HD / 16, P = Lds<HD>::P, TP = Lds<HD>::TP, TILE = 16 * TP, KP6 = Lds<HD>::KP6;
  const int NW = blockDim.x >> 6, D = H * HD;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bool active = w < at.nb;
  const int i = 16 * w + c;  // this lane's query slot, and its key slot
  // The wave's own q and dO rows: held in registers across the steps, or at
  // head_dim 64 and up re-read from LDS in each step (32+ fewer registers,
  // which is what lets two workgroups share a CU there).
  // With SPL (V staged as split rows) dP^T runs on the bf16 matrix cores
  // from dO split once here.
  constexpr bool QG_LDS = HD >= 64;
  static_assert(!SPL || (!QG_LDS && HD % 32 == 0), "split dP^T: head_dim 32");
  float q[QG_LDS ? 1 : W], go[QG_LDS || SPL ? 1 : W], dqi = 0.f;
  u4 gos[SPL ? 3 * (W / 8) : 1];
  if (active) {
    float qa[W], ga[W];
    lds_get<W>(Qs + i * P + g * W, qa);
    lds_get<W>(Gs + i * P + g * W, ga);
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < W; ++t) d += ga[t] * oo[t];
    dqi = sum_g(d);  // Dq = dO . O of query i
    if constexpr (SPL) {
#pragma unroll
      for (int kc = 0; kc < W / 8; ++kc) split8(ga + 8 * kc, gos + 3 * kc);
    }
    if constexpr (!QG_LDS) {
#pragma unroll
      for (int t = 0; t < W; ++t) {
        q[t] = qa[t];
        if constexpr (!SPL) go[t] = ga[t];
      }
    }
  }
  f4 dq[DT], dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  const int nb = at.nb;
  // A query with no live key (li = 0) or a key with log cf kOff gets an
  // exponent near -1e30, so exp gives 0 exactly without a test per key.
  const float mie = li > 0.f ? mi : 1e30f;
  float* const Tb1 = Tb + mul24(NW * 2, TILE);  // the second tile buffer
  // Phase 1 of step s: tile (query block w, key block J = (w + s) mod nb):
  // S^T and dP^T, then A and dS, the dQ share, and A, dS left in LDS.
  auto phase1 = [&](int s, bool v_staged) {
    float* tb = nbuf == 2 && (s & 1) ? Tb1 : Tb;
    int J = w + s;
    if (J >= nb) J -= nb;
    f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
    if constexpr (SPL) {  // V staged split: v_staged holds
      float k[W];
      lds_get<W>(Ks + mul24(16 * J + c, P) + g * W, k);
      const unsigned* vb = reinterpret_cast<const unsigned*>(Vs) + mul24(16 * J + c, KP6) + g * (W / 8) * 12;
#pragma unroll
      for (int t = 0; t < W; ++t) st = mfma(k[t], q[t], st);
#pragma unroll
      for (int kc = 0; kc < W / 8; ++kc) {
        u4 a[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) a[p] = *reinterpret_cast<const u4*>(vb + kc * 12 + 4 * p);
        dp = mfma6(a, gos + 3 * kc, dp);
      }
    } else {
      float k[W], v[W];
      lds_get<W>(Ks + mul24(16 * J + c, P) + g * W, k);
      if (v_staged)
        lds_get<W>(Vs + mul24(16 * J + c, P) + g * W, v);
      else if (16 * J + c < at.cnt)
        qkv_get<W, XF>(qkv, ldq, at.row(16 * J + c), 2 * D + at.h * HD + g * W, xf, v);  // chunk rows
      else
#pragma unroll
        for (int t = 0; t < W; ++t) v[t] = 0.f;
      if constexpr (QG_LDS) {
        float qa[W], ga[W];
        lds_get<W>(Qs + i * P + g * W, qa);
        lds_get<W>(Gs + i * P + g * W, ga);
#pragma unroll
        for (int t = 0; t < W; ++t) st = mfma(k[t], qa[t], st), dp = mfma(v[t], ga[t], dp);
      } else {
#pragma unroll
        for (int t = 0; t < W; ++t) st = mfma(k[t], q[t], st), dp = mfma(v[t], go[t], dp);
      }
    }
    float lc[4], a[4], ds[4];
    lds_get<4>(lcf + 16 * J + 4 * g, lc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // query i, key 16J + 4g + r
      a[r] = __expf(st[r] * sc + lc[r] - mie) * li;
      ds[r] = a[r] * (dp[r] - dqi);
    }
    // dQ^T += K^T dS^T over the tile's keys.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float kk[DT];
      lds_get<DT>(Ks + mul24(16 * J + 4 * g + r, P) + c * DT, kk);
#pragma unroll
      for (int t = 0; t < DT; ++t) dq[t] = mfma(kk[t], ds[r], dq[t]);
    }
    float* ta = tb + mul24(2 * w, TILE);
    *reinterpret_cast<float4*>(ta + c * TP + 4 * g) = make_float4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<float4*>(ta + TILE + c * TP + 4 * g) = make_float4(ds[0], ds[1], ds[2], ds[3]);
  };
  // Phase 2 of step s: key block w's tile from query block Ip = (w - s) mod nb:
  // dK^T += Q^T dS, dV^T += dO^T A, and the key's dS summed.
  auto phase2 = [&](int s) {
    const float* tb = nbuf == 2 && (s & 1) ? Tb1 : Tb;
    int Ip = w - s;
    if (Ip < 0) Ip += nb;
    const float* ta = tb + mul24(2 * Ip, TILE);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float av = ta[(4 * g + r) * TP + c], dsv = ta[TILE + (4 * g + r) * TP + c];
      cfa += dsv;
      float qq[DT], gg[DT];
      lds_get<DT>(Qs + mul24(16 * Ip + 4 * g + r, P) + c * DT, qq);
      lds_get<DT>(Gs + mul24(16 * Ip + 4 * g + r, P) + c * DT, gg);
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

// One item per workgroup: the item's slices, its own rows' O and statistics
// loaded into registers, staged in LDS, one barrier, then its backward.
template <int HD, int MAXT, bool XF = false, bool SPL = false>
__global__ void __launch_bounds__(MAXT) attn_bwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                        const int* __restrict__ off, int N, int n0, int64_t eb,
                                                        int S, int H, float sc, const float* __restrict__ dmerged,
                                                        int64_t ldg, const float* __restrict__ merged, int64_t ldm,
                                                        const float* __restrict__ ml,
                                                        const float* __restrict__ cf_seq, int64_t ldc,
                                                        float* __restrict__ qkv_adj, int64_t lda,
                                                        float* __restrict__ cfh, int nbuf, int vlds, QkvXf xf) {
  constexpr int W = HD / 4, P = Lds<HD>::P, KP6 = Lds<HD>::KP6;
  extern __shared__ float lds[];
  const int NW = blockDim.x >> 6, R = NW * 16, D = H * HD;
  float* Qs = lds;
  float* Ks = Qs + R * P;
  float* Gs = Ks + R * P;
  float* Vs = Gs + R * P;  // when vlds: fp32 rows, or split rows with SPL (which needs vlds)
  float* lcf = Vs + (vlds ? R * (SPL ? KP6 : P) : 0);
  float* Tb = lcf + R;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 4, i = 16 * w + (l & 15);
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, n0, eb);
  float oo[W], mi = kOff, li = 0.f;
  // Each wave stages its own block -- rows 16w .. 16w+15 of Q, K, dO (and V),
  // lane (c, g) the slice of row 16w + c that is its MFMA operand -- and the
  // cf of its own keys. Step 0 of the tile schedule (tile (w, w)) reads only
  // that block, so a wave starts computing as soon as its own loads are in,
  // and the first workgroup barrier comes after step 0, not before it.
  if (w < at.nb) {
    float q[W], k[W], go[W], v[W];
    const bool real = i < at.cnt;
    if (real) {
      const size_t r = at.row(i);
      qkv_get<W, XF>(qkv, ldq, r, at.h * HD + g * W, xf, q);
      qkv_get<W, XF>(qkv, ldq, r, D + at.h * HD + g * W, xf, k);
      gmem_get<W>(dmerged + r * ldg + at.h * HD + g * W, go);
      if (vlds) qkv_get<W, XF>(qkv, ldq, r, 2 * D + at.h * HD + g * W, xf, v);
      gmem_get<W>(merged + at.grow(i) * ldm + at.h * HD + g * W, oo);  // the whole's rows
      const float* m2 = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
      mi = m2[0], li = m2[1];
    } else {
#pragma unroll
      for (int t = 0; t < W; ++t) q[t] = k[t] = go[t] = v[t] = oo[t] = 0.f;
    }
    const float pcf = real && g == 0 ? cf_seq[size_t(at.n) * ldc + i] : 0.f;
    float* o = Qs + i * P + g * W;
#pragma unroll
    for (int t = 0; t < W; t += 4) {
      *reinterpret_cast<float4*>(o + t) = make_float4(q[t], q[t + 1], q[t + 2], q[t + 3]);
      *reinterpret_cast<float4*>(o + (Ks - Qs) + t) = make_float4(k[t], k[t + 1], k[t + 2], k[t + 3]);
      *reinterpret_cast<float4*>(o + (Gs - Qs) + t) = make_float4(go[t], go[t + 1], go[t + 2], go[t + 3]);
      if (!SPL && vlds)
        *reinterpret_cast<float4*>(o + (Vs - Qs) + t) = make_float4(v[t], v[t + 1], v[t + 2], v[t + 3]);
    }
    if constexpr (SPL) {
      unsigned* ov = reinterpret_cast<unsigned*>(Vs) + i * KP6 + g * (W / 8) * 12;
#pragma unroll
      for (int kc = 0; kc < W / 8; ++kc) {
        u4 vp[3];
        split8(v + 8 * kc, vp);
#pragma unroll
        for (int p = 0; p < 3; ++p) *reinterpret_cast<u4*>(ov + kc * 12 + 4 * p) = vp[p];
      }
    }
    if (g == 0) lcf[i] = pcf > 0.f ? log_cf(pcf) : kOff;
  }
  BwdOut<HD> out;
  bwd_item<HD, XF, SPL>(at, Qs, Ks, Gs, Vs, lcf, Tb, nbuf, vlds, oo, mi, li, qkv, ldq, xf, H, sc, out);
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
  // the old value loaded with cf (in bounds either way), so that it does not
  // wait on cf's test; the heads' loads issued eight at a time, then summed in
  // head order
  float* out = cf_seq_adj + int64_t(n) * ldca + k;
  const float old = *out;
  const float* p = cfh + int64_t(n) * H * S + k;
  float total = 0.f;
  int hh = 0;
  for (; hh + 8 <= H; hh += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[int64_t(hh + u) * S];
#pragma unroll
    for (int u = 0; u < 8; ++u) total += v[u];
  }
  for (; hh < H; ++hh) total += p[int64_t(hh) * S];
  if (cf > 0.f) *out = old + total / cf;
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

// The inverse scales [blocks][T] of a capacity's dead rows (block pairs of
// qkv_adj, whose pairs zero_dead_kernel clears) set to 0.
__global__ void zero_dead_inv_kernel(float* __restrict__ inv, int blocks, int N, int T, const int* __restrict__ off) {
  const int64_t first = int64_t(N) + off[N];
  const int64_t rows = int64_t(T) - first;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < rows * blocks;
       i += int64_t(gridDim.x) * blockDim.x)
    inv[(i / rows) * T + first + i % rows] = 0.f;
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
  if (sh->head_dim < 1 || sh->head_dim > 128) return PET_ATTN_EHEADDIM;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (int64_t(sh->n_rows) * 3 * D >= (int64_t(1) << 31) * 4) return PET_ATTN_EINDEX;
  if (int64_t(sh->n_atoms) * sh->heads * sh->slots >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  return PET_ATTN_OK;
}
// A matrix argument: non-null, rows no narrower than width, and 16-byte
// aligned rows unless head_dim is not a multiple of 4 (the streaming kernels
// then load columns one at a time: 4-byte alignment).
int check_matrix(const void* p, int64_t ld, int64_t width, int head_dim) {
  if (!p || ld < width) return PET_ATTN_EINVAL;
  if (head_dim % 4 != 0) return (reinterpret_cast<uintptr_t>(p) & 3u) ? PET_ATTN_EALIGN : PET_ATTN_OK;
  if (!aligned16(p) || ld % 4 != 0) return PET_ATTN_EALIGN;
  return PET_ATTN_OK;
}
int check_run(const pet_attn_shape* sh, int n0, int n1, int e0) {
  if (n0 < 0 || n1 < n0 || n1 > sh->n_atoms || e0 < 0) return PET_ATTN_EINVAL;
  return PET_ATTN_OK;
}
int waves_for(int S) { return (S + 15) / 16; }

// Process-wide tuning options (pet_attn_set_option): each an atomic read
// once per launch, never the environment.
std::atomic<int> g_options[PET_OPT_COUNT] = {{0}, {1}, {0}, {0}, {0}, {6}, {0}, {0}, {0}, {1}};
int option(int o) { return g_options[o].load(std::memory_order_relaxed); }
bool split_enabled() { return option(PET_OPT_SPLIT) != 0; }

// Per-kernel facts the launchers consult on every call, looked up once: the
// compiled VGPR count, and (per device) the dynamic LDS limit already raised.
std::mutex g_kernel_mu;
int kernel_vgprs(const void* k) {
  static std::map<const void*, int> vgprs;
  std::lock_guard<std::mutex> lock(g_kernel_mu);
  auto it = vgprs.find(k);
  if (it != vgprs.end()) return it->second;
  hipFuncAttributes fa{};
  const int v = hipFuncGetAttributes(&fa, k) == hipSuccess ? fa.numRegs : -1;
  vgprs[k] = v;
  return v;
}
template <class K>
void allow_lds(K k, size_t bytes) {
  if (bytes <= 65536) return;
  static std::map<std::pair<int, const void*>, size_t> raised;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  const void* kp = reinterpret_cast<const void*>(k);
  std::lock_guard<std::mutex> lock(g_kernel_mu);
  size_t& have = raised[{dev, kp}];
  if (have >= bytes) return;
  if (hipFuncSetAttribute(kp, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) == hipSuccess) have = bytes;
}

// Workgroups of kernel k (NW waves, lds bytes of LDS) one CU holds at once,
// by the rules measured on gfx950 with spin kernels: a SIMD holds
// min(8, 512 / vgprs) waves (vgprs rounded up to 8); workgroups whose wave
// count is not a multiple of 4 lose a wave slot a SIMD in the packing,
// floor((4c - 4) / NW) of them a CU (c waves a SIMD), else floor(4c / NW);
// LDS goes in 2 KB granules of 160 KB. (The runtime's occupancy query counts
// more than fit for 5-wave workgroups.)
int resident_wgs(const void* k, int NW, size_t lds) {
  const int regs = kernel_vgprs(k);
  if (regs < 0) return 1;
  const int vg = std::max(8, (regs + 7) / 8 * 8);
  const int c = std::min(8, 512 / vg);
  const int by_vgpr = NW % 4 ? (4 * c - 4) / NW : 4 * c / NW;
  const size_t gran = (lds + 2047) / 2048 * 2048;
  const int by_lds = gran ? int(163840 / gran) : 8;
  return std::max(1, std::min(by_vgpr, by_lds));
}

// Which kernel a launch takes (the LDS-staged kernels; the streaming ones are
// chosen before, by streams()): its LDS bytes, its split products and, for the
// backward, its LDS layout. Made by plan_fwd / plan_bwd from the shape and
// the options, so that a caller can ask (pet_attn_describe) what a launch runs.
struct Plan {
  int ok = 0;             // 0: the shape does not fit the staged kernels' LDS
  size_t bytes = 0;       // dynamic LDS
  bool split = false;     // forward: the scores; backward: dP, on the bf16 matrix cores
  bool valu = false;      // forward: the vector-ALU kernel
  int vlds = 0, nbuf = 0; // backward: V staged, tile buffers
  bool pair = false;      // backward: the fp16-pair kernel (attention_pair.hip)
  int resident = 0;       // workgroups a CU
};

// The fp16-pair forward and backward (attention_pair.hip), head_dim 32.
size_t pair_fwd_bytes(int HD, int NW);
const void* pair_fwd_kernel_ptr(int HD);
int pair_fwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
             const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, hipStream_t st);
size_t pair_bwd_bytes(int HD, int NW);
const void* pair_bwd_kernel_ptr(int HD);
int pair_bwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
             const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
             const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, hipStream_t st,
             void* qpairs = nullptr, int64_t prows = 0);

template <int HD>
Plan plan_fwd(const pet_attn_shape& sh, bool xf) {
  Plan p;
  const int NW = waves_for(sh.slots);
  const size_t cap = size_t(max_lds_bytes());
  p.bytes = sizeof(float) * Lds<HD>::fwd_floats(NW);
  if (p.bytes > cap) return p;
  p.ok = 1;
  const void* plain = reinterpret_cast<const void*>(attn_fwd_kernel<HD, 512, false, false>);
  p.resident = resident_wgs(plain, NW, p.bytes);
  // scores on the bf16 matrix cores (split fp32) where head_dim is a multiple
  // of 32 and the split K rows fit as many workgroups a CU; option PET_OPT_SPLIT 0
  // keeps every product on the fp32 matrix cores
  if constexpr (HD % 32 == 0) {
    const size_t sbytes = sizeof(float) * Lds<HD>::fwd_floats(NW, true);
    if (split_enabled() && sbytes <= cap) {
      const void* split = reinterpret_cast<const void*>(attn_fwd_kernel<HD, 512, false, true>);
      const int r = resident_wgs(split, NW, sbytes);
      if (r >= p.resident) p.split = true, p.bytes = sbytes, p.resident = r;
    }
  }
  if constexpr (HD == 32 || HD == 64) {  // the fp16-pair forward (attention_pair.hip) unless an option asks otherwise
    const size_t pb = pair_fwd_bytes(HD, NW);
    if (split_enabled() && option(PET_OPT_FWD_KERNEL) == 0 && pb <= cap)
      p.pair = true, p.split = false, p.bytes = pb, p.resident = resident_wgs(pair_fwd_kernel_ptr(HD), NW, pb);
  }
  if constexpr (HD <= 64) {  // option PET_OPT_FWD_KERNEL 3: the vector-ALU kernel, for comparison
    const int threads = 64 * ((sh.slots + 63) / 64);
    const size_t vb = sizeof(float) * (size_t(2) * threads * HD + threads);
    if (option(PET_OPT_FWD_KERNEL) == 3 && !xf && threads <= 256 && vb <= cap)
      p.valu = true, p.split = false, p.pair = false, p.bytes = vb, p.resident = 0;
  }
  return p;
}

// The forward over atoms [n0, n1), qkv a chunk whose edge 0 is row eb.
template <int HD>
int launch_fwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, hipStream_t st) {
  const bool x = xf.rs || xf.b;
  const Plan p = plan_fwd<HD>(sh, x);
  if (!p.ok) return PET_ATTN_ESLOTS;
  const int NW = waves_for(sh.slots);
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  if constexpr (HD <= 64) {
    if (p.valu) {
      const int threads = 64 * ((sh.slots + 63) / 64);
      allow_lds(attn_fwd_valu_kernel<HD>, p.bytes);
      hipLaunchKernelGGL(attn_fwd_valu_kernel<HD>, dim3(unsigned(items)), dim3(threads), p.bytes, st, qkv, ldq, off,
                         sh.n_atoms, n0, eb, sh.slots, sh.heads, sh.scale, cf_seq, ldc, merged, ldm, ml);
      return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
    }
  }
  if (p.pair) return pair_fwd(sh, n0, n1, eb, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, xf, st);
  using KT = decltype(&attn_fwd_kernel<HD, 512, false, false>);
  KT k;
  if constexpr (HD % 32 == 0) {
    if (p.split)
      k = NW <= 8 ? (x ? attn_fwd_kernel<HD, 512, true, true> : attn_fwd_kernel<HD, 512, false, true>)
                  : (x ? attn_fwd_kernel<HD, 1024, true, true> : attn_fwd_kernel<HD, 1024, false, true>);
    else
      k = NW <= 8 ? (x ? attn_fwd_kernel<HD, 512, true> : attn_fwd_kernel<HD, 512, false>)
                  : (x ? attn_fwd_kernel<HD, 1024, true> : attn_fwd_kernel<HD, 1024, false>);
  } else {
    k = NW <= 8 ? (x ? attn_fwd_kernel<HD, 512, true> : attn_fwd_kernel<HD, 512, false>)
                : (x ? attn_fwd_kernel<HD, 1024, true> : attn_fwd_kernel<HD, 1024, false>);
  }
  allow_lds(k, p.bytes);
  hipLaunchKernelGGL(k, dim3(unsigned(items)), dim3(64 * NW), p.bytes, st, qkv, ldq, off, sh.n_atoms, n0, eb,
                     sh.slots, sh.heads, sh.scale, cf_seq, ldc, merged, ldm, ml, xf);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

// The fullest layout that fits (V staged and two tile buffers, else V from
// global memory, else also one tile buffer) -- unless it leaves one workgroup
// a CU and a leaner one fits more: then the leaner. Measured on MI355X: at
// head_dim 32 the fullest is fastest though the leanest would fit a third
// workgroup (C3 backward 429 us against 466-493 us); at head_dim 64 the
// fullest holds one workgroup a CU and V-from-global with one buffer two (C5
// backward 3853 -> 3244 us). The options PET_OPT_BWD_VLDS (1 staged, 2 not)
// and PET_OPT_BWD_NBUF (1, 2) force a layout where it fits. dP^T runs on the
// bf16 matrix cores (V staged split) at head_dim 32 when V is staged and the
// split rows keep as many workgroups a CU.
template <int HD>
Plan plan_bwd(const pet_attn_shape& sh) {
  Plan p;
  const int NW = waves_for(sh.slots);
  const void* k = reinterpret_cast<const void*>(attn_bwd_kernel<HD, 512, false>);
  const int force_v = option(PET_OPT_BWD_VLDS), force_b = option(PET_OPT_BWD_NBUF);
  const size_t cap = size_t(max_lds_bytes());
  const int layouts[3][2] = {{1, 2}, {0, 2}, {0, 1}};  // (vlds, nbuf), fullest first
  int best = -1, best_res = 0;
  for (int j = 0; j < 3; ++j) {
    const size_t b = sizeof(float) * Lds<HD>::bwd_floats(NW, layouts[j][1], layouts[j][0]);
    if (b > cap) continue;
    const int res = resident_wgs(k, NW, b);
    if (best < 0) {
      best = j, best_res = res;
      if (res > 1) break;  // the fullest that fits holds more than one: keep it
    } else if (res > best_res) {
      best = j, best_res = res;
    }
  }
  if (best < 0) return p;
  p.ok = 1;
  p.vlds = layouts[best][0], p.nbuf = layouts[best][1], p.resident = best_res;
  p.bytes = sizeof(float) * Lds<HD>::bwd_floats(NW, p.nbuf, p.vlds);
  if (force_v || force_b) {
    const int v = force_v ? (force_v == 1) : p.vlds, b = force_b ? force_b : p.nbuf;
    const size_t fb = sizeof(float) * Lds<HD>::bwd_floats(NW, b, v);
    if ((b == 1 || b == 2) && fb <= cap) p.vlds = v, p.nbuf = b, p.bytes = fb, p.resident = resident_wgs(k, NW, fb);
  }
  if constexpr (HD == 32 || HD == 64) {
    // every product as fp16 pairs (attention_pair.hip) unless an option asks
    // for the tile-exchange kernel or for fp32 products only
    const size_t pb = pair_bwd_bytes(HD, NW);
    if (split_enabled() && option(PET_OPT_BWD_KERNEL) == 0 && !force_v && !force_b && pb <= cap) {
      p.pair = true, p.vlds = 0, p.nbuf = 2, p.bytes = pb, p.resident = resident_wgs(pair_bwd_kernel_ptr(HD), NW, pb);
      return p;
    }
  }
  if constexpr (HD == 32) {
    const size_t sb = sizeof(float) * Lds<HD>::bwd_floats(NW, p.nbuf, true, true);
    if (p.vlds && split_enabled() && sb <= cap) {
      const void* ks = reinterpret_cast<const void*>(attn_bwd_kernel<HD, 512, false, true>);
      const int r = resident_wgs(ks, NW, sb);
      if (r >= p.resident) p.split = true, p.bytes = sb, p.resident = r;
    }
  }
  return p;
}

// The backward over atoms [n0, n1); qkv, dmerged and qkv_adj are the chunk's.
template <int HD>
int launch_bwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
               const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, hipStream_t st) {
  const Plan p = plan_bwd<HD>(sh);
  if (!p.ok) return PET_ATTN_ESLOTS;
  const int NW = waves_for(sh.slots);
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  if (p.pair)
    return pair_bwd(sh, n0, n1, eb, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, xf,
                    st);
  const bool x = xf.rs || xf.b;
  auto k = NW <= 8 ? (x ? attn_bwd_kernel<HD, 512, true> : attn_bwd_kernel<HD, 512, false>)
                   : (x ? attn_bwd_kernel<HD, 1024, true> : attn_bwd_kernel<HD, 1024, false>);
  if constexpr (HD == 32) {
    if (p.split)
      k = NW <= 8 ? (x ? attn_bwd_kernel<HD, 512, true, true> : attn_bwd_kernel<HD, 512, false, true>)
                  : (x ? attn_bwd_kernel<HD, 1024, true, true> : attn_bwd_kernel<HD, 1024, false, true>);
  }
  allow_lds(k, p.bytes);
  hipLaunchKernelGGL(k, dim3(unsigned(items)), dim3(64 * NW), p.bytes, st, qkv, ldq, off, sh.n_atoms, n0, eb,
                     sh.slots, sh.heads, sh.scale, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh,
                     p.nbuf, p.vlds, xf);
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

int cf_adjoint(const pet_attn_shape& sh, const float* cfh, const float* cf_seq, int64_t ldc, float* cf_seq_adj,
               int64_t ldca, hipStream_t st) {
  const int64_t NS = int64_t(sh.n_atoms) * sh.slots;
  if (NS == 0) return PET_ATTN_OK;
  hipLaunchKernelGGL(attn_cf_adjoint_kernel, dim3(unsigned((NS + 255) / 256)), dim3(256), 0, st, cfh, cf_seq, ldc,
                     cf_seq_adj, ldca, sh.n_atoms, sh.slots, sh.heads);
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
    case PET_ATTN_EHEADDIM: return "unsupported head_dim (1 to 128)";
    case PET_ATTN_ESLOTS: return "too many slots per atom";
    case PET_ATTN_EALIGN: return "a pointer or leading dimension is not a multiple of 4 floats";
    case PET_ATTN_ELAUNCH: return "a HIP launch or runtime call failed";
    case PET_ATTN_EBLAS: return "the BLAS call of a linear failed";
    case PET_ATTN_EWORKSPACE: return "workspace smaller than the matching *_workspace() size";
    case PET_ATTN_EINDEX: return "an index does not fit 2^31";
    case PET_ATTN_ESCRATCH:
      return "N * heads * slots is above pet_attn_bwd_noalloc's scratch (PET_ATTN_NOALLOC_MAX_SCRATCH bytes)";
    case 20: return "a tensor the model's architecture needs is missing";
    case 21: return "a tensor's shape disagrees with the model's hyperparameters";
    case 22: return "a device allocation failed";
    default: return "unknown pet_attn error";
  }
}

int pet_attn_set_option(int opt, int value) {
  if (opt <= 0 || opt >= PET_OPT_COUNT) return PET_ATTN_EINVAL;
  static const int lo[PET_OPT_COUNT] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, hi[PET_OPT_COUNT] = {0, 1, 3, 2, 2, 6, 1, 1, 2, 1};
  if (value < lo[opt] || value > hi[opt]) return PET_ATTN_EINVAL;
  g_options[opt].store(value, std::memory_order_relaxed);
  return PET_ATTN_OK;
}

int pet_attn_get_option(int opt) { return opt > 0 && opt < PET_OPT_COUNT ? option(opt) : -1; }

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

}  // extern "C"

namespace pet_attn {
// The streaming kernels (attention_stream.hip): any S, any head_dim 1..128.
int stream_fwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, hipStream_t st);
int stream_bwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
               const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, hipStream_t st);
// The LDS-staged kernels take head_dim a multiple of 16 and S within their LDS
// envelope; everything else streams (or everything, with PET_OPT_ATTN_STREAM).
bool streams(const pet_attn_shape& sh) {
  return sh.head_dim % 16 != 0 || option(PET_OPT_ATTN_STREAM) != 0 || sh.slots > pet_attn_max_slots(sh.head_dim);
}
}  // namespace pet_attn

extern "C" int pet_attn_describe(const pet_attn_shape* sh, pet_attn_plan* out) {
  if (!out) return PET_ATTN_EINVAL;
  *out = pet_attn_plan{};
  if (int e = check_shape(sh)) return e;
  if (streams(*sh)) {
    out->streaming = 1;
    return PET_ATTN_OK;
  }
  return with_head_dim(sh->head_dim, [&](auto hd) {
    constexpr int HD = decltype(hd)::value;
    const Plan f = plan_fwd<HD>(*sh, false), b = plan_bwd<HD>(*sh);
    out->fwd_split_scores = f.split, out->fwd_valu = f.valu, out->fwd_lds_bytes = int(f.bytes);
    out->fwd_workgroups_per_cu = f.resident;
    out->bwd_split_dp = b.split, out->bwd_v_staged = b.vlds, out->bwd_tile_buffers = b.nbuf;
    out->bwd_lds_bytes = int(b.bytes), out->bwd_workgroups_per_cu = b.resident, out->bwd_pair = b.pair, out->fwd_pair = f.pair;
    out->waves = waves_for(sh->slots);
    return PET_ATTN_OK;
  });
}

namespace {
int fwd_run(const pet_attn_shape* sh, int n0, int n1, int e0, const float* qkv, int64_t ldq, const int* off,
            const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (int e = check_run(sh, n0, n1, e0)) return e;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (n1 == n0) return PET_ATTN_OK;
  if (int e = check_matrix(qkv, ldq, 3 * D, sh->head_dim)) return e;
  if (int e = check_matrix(merged, ldm, D, sh->head_dim)) return e;
  if (!off || !cf_seq || ldc < sh->slots) return PET_ATTN_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t eb = int64_t(n1 - n0) - e0;
  if (streams(*sh)) return stream_fwd(*sh, n0, n1, eb, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, xf, st);
  return with_head_dim(sh->head_dim, [&](auto hd) {
    return launch_fwd<decltype(hd)::value>(*sh, n0, n1, eb, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, xf, st);
  });
}

int bwd_run(const pet_attn_shape* sh, int n0, int n1, int e0, const float* qkv, int64_t ldq, const int* off,
            const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq,
            int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (int e = check_run(sh, n0, n1, e0)) return e;
  const int64_t D = int64_t(sh->heads) * sh->head_dim;
  if (n1 == n0) return PET_ATTN_OK;
  if (int e = check_matrix(qkv, ldq, 3 * D, sh->head_dim)) return e;
  if (int e = check_matrix(dmerged, ldg, D, sh->head_dim)) return e;
  if (int e = check_matrix(merged, ldm, D, sh->head_dim)) return e;
  if (int e = check_matrix(qkv_adj, lda, 3 * D, sh->head_dim)) return e;
  if (!off || !ml || !cf_seq || !cfh || ldc < sh->slots) return PET_ATTN_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t eb = int64_t(n1 - n0) - e0;
  if (streams(*sh))
    return stream_bwd(*sh, n0, n1, eb, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh,
                      xf, st);
  return with_head_dim(sh->head_dim, [&](auto hd) {
    return launch_bwd<decltype(hd)::value>(*sh, n0, n1, eb, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq,
                                           ldc, qkv_adj, lda, cfh, xf, st);
  });
}

int fwd_whole(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* cf_seq,
              int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  // the whole matrix is the run of every atom: own rows first, edge 0 at row N
  if (int e = fwd_run(sh, 0, sh->n_atoms, 0, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, xf, stream)) return e;
  return zero_dead(merged, ldm, sh->heads * sh->head_dim, *sh, off, reinterpret_cast<hipStream_t>(stream));
}

int bwd_whole(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* dmerged,
              int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
              float* qkv_adj, int64_t lda, float* cfh, float* cf_seq_adj, int64_t ldca, QkvXf xf, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  if (!cf_seq_adj || ldca < sh->slots) return PET_ATTN_EINVAL;
  if (int e = bwd_run(sh, 0, sh->n_atoms, 0, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda,
                      cfh, xf, stream))
    return e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int e = cf_adjoint(*sh, cfh, cf_seq, ldc, cf_seq_adj, ldca, st)) return e;
  return zero_dead(qkv_adj, lda, 3 * sh->heads * sh->head_dim, *sh, off, st);
}
}  // namespace

// The core's backward as pet_attn_bwd_xf, with qkv_adj written as block pairs
// into qpairs instead of fp32: T rows of 3D / 8 groups of 8 values (hi then lo
// fp16, 16 bytes each), each (row, head, q | k | v) slice of head_dim values
// scaled by its own power of two, then the slices' inverse scales [3H][T]
// (block m H + h): the A operand, K blocks of head_dim, of the product that
// reads qkv_adj next (pet_gemm_nt_pp_blocks). Dead rows hold zeros. Only
// where the fp16-pair backward takes the shape and 3H is at most 32; else
// PET_ATTN_ESLOTS, and the caller takes the fp32 form.
int pet_attn_bwd_xf_blocks(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const float* rs, const float* b,
                           const int* off, const float* dmerged, int64_t ldg, const float* merged, int64_t ldm,
                           const float* ml, const float* cf_seq, int64_t ldc, void* qpairs, float* cfh,
                           float* cf_seq_adj, int64_t ldca, hipStream_t st) {
  using namespace pet_attn;
  if (int e = check_shape(sh)) return e;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  if (!cf_seq_adj || ldca < sh->slots || !qpairs || !aligned16(qpairs)) return PET_ATTN_EINVAL;
  const int HD = sh->head_dim;
  if (streams(*sh) || (HD != 32 && HD != 64) || 3 * sh->heads > 32) return PET_ATTN_ESLOTS;
  const bool pair = HD == 32 ? plan_bwd<32>(*sh).pair : plan_bwd<64>(*sh).pair;
  if (!pair) return PET_ATTN_ESLOTS;
  const int64_t D = int64_t(sh->heads) * HD, T = sh->n_rows;
  if (int e = check_matrix(qkv, ldq, 3 * D, HD)) return e;
  if (int e = check_matrix(dmerged, ldg, D, HD)) return e;
  if (int e = check_matrix(merged, ldm, D, HD)) return e;
  if (!off || !ml || !cf_seq || !cfh || ldc < sh->slots) return PET_ATTN_EINVAL;
  if (int e = pair_bwd(*sh, 0, sh->n_atoms, sh->n_atoms, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc,
                       nullptr, 0, cfh, QkvXf{rs, b}, st, qpairs, T))
    return e;
  if (int e = cf_adjoint(*sh, cfh, cf_seq, ldc, cf_seq_adj, ldca, st)) return e;
  if (!sh->dead || sh->n_rows == sh->n_atoms) return PET_ATTN_OK;
  if (int e = zero_dead(static_cast<float*>(qpairs), 3 * D, int(3 * D), *sh, off, st)) return e;
  hipLaunchKernelGGL(zero_dead_inv_kernel, dim3(256), dim3(256), 0, st,
                     reinterpret_cast<float*>(static_cast<char*>(qpairs) + size_t(T) * 3 * D * 4), 3 * sh->heads,
                     sh->n_atoms, sh->n_rows, off);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

extern "C" {

int pet_attn_fwd_run(const pet_attn_shape* sh, int n0, int n1, int e0, const float* qkv, int64_t ldq, const int* off,
                     const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, void* stream) {
  return fwd_run(sh, n0, n1, e0, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, QkvXf{}, stream);
}

int pet_attn_bwd_run(const pet_attn_shape* sh, int n0, int n1, int e0, const float* qkv, int64_t ldq, const int* off,
                     const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
                     const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, void* stream) {
  return bwd_run(sh, n0, n1, e0, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh,
                 QkvXf{}, stream);
}

int pet_attn_cf_adjoint(const pet_attn_shape* sh, const float* cfh, const float* cf_seq, int64_t ldc,
                        float* cf_seq_adj, int64_t ldca, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (!cfh || !cf_seq || !cf_seq_adj || ldc < sh->slots || ldca < sh->slots) return PET_ATTN_EINVAL;
  return cf_adjoint(*sh, cfh, cf_seq, ldc, cf_seq_adj, ldca, reinterpret_cast<hipStream_t>(stream));
}

int pet_attn_zero_dead(const pet_attn_shape* sh, float* x, int64_t ld, int width, const int* off, void* stream) {
  if (int e = check_shape(sh)) return e;
  if (!x || !off || width < 1 || ld < width) return PET_ATTN_EINVAL;
  return zero_dead(x, ld, width, *sh, off, reinterpret_cast<hipStream_t>(stream));
}

int pet_attn_fwd(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* cf_seq,
                 int64_t ldc, float* merged, int64_t ldm, float* ml, void* stream) {
  return fwd_whole(sh, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, QkvXf{}, stream);
}

int pet_attn_bwd(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off, const float* dmerged,
                 int64_t ldg, const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
                 float* qkv_adj, int64_t lda, float* cfh, float* cf_seq_adj, int64_t ldca, void* stream) {
  return bwd_whole(sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, cf_seq_adj, ldca,
                   QkvXf{}, stream);
}

}  // extern "C"

// ---- the allocation-free backward ---------------------------------------------
// pet_attn_bwd_noalloc's cfh scratch: a file-scope device array, one per GPU
// the library runs on, held until the process ends. Host code never uses the
// array's name as an address (on the host it is a stand-in symbol): each
// device's address is looked up once, with that device current, by
// hipGetSymbolAddress, and kept here.
namespace pet_attn {
constexpr int64_t kScratchFloats = PET_ATTN_NOALLOC_MAX_SCRATCH / sizeof(float);
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's scratch address (null if it cannot be found).
float* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch[dev].load(std::memory_order_relaxed);
  if (p) return p;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) {
    (void) hipGetLastError();
    return nullptr;
  }
  p = static_cast<float*>(addr);
  g_scratch[dev].store(p, std::memory_order_release);
  return p;
}
}  // namespace pet_attn

extern "C" {

int pet_attn_bwd_noalloc(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off,
                         const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
                         const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cf_seq_adj,
                         int64_t ldca, void* stream) {
  if (int e = check_shape(sh)) return e;
  // cfh [N, H, S] in the scratch array: every element the backward writes,
  // nothing read before it is written, so nothing needs clearing
  if (int64_t(sh->n_atoms) * sh->heads * sh->slots > kScratchFloats) return PET_ATTN_ESCRATCH;
  if (sh->n_atoms == 0) return PET_ATTN_OK;
  float* cfh = scratch_ptr();
  if (!cfh) return PET_ATTN_ELAUNCH;
  return bwd_whole(sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, cf_seq_adj, ldca,
                   QkvXf{}, stream);
}

int pet_attn_fwd_xf(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const float* row_scale,
                    const float* bias, const int* off, const float* cf_seq, int64_t ldc, float* merged, int64_t ldm,
                    float* ml, void* stream) {
  return fwd_whole(sh, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml, QkvXf{row_scale, bias}, stream);
}

int pet_attn_bwd_xf(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const float* row_scale,
                    const float* bias, const int* off, const float* dmerged, int64_t ldg, const float* merged,
                    int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda,
                    float* cfh, float* cf_seq_adj, int64_t ldca, void* stream) {
  return bwd_whole(sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, cf_seq_adj, ldca,
                   QkvXf{row_scale, bias}, stream);
}

}  // extern "C"
