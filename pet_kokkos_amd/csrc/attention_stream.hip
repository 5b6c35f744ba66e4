// PET's per-atom attention for any slot count S and any head_dim 1..128: the
// streaming kernels. The LDS-staged kernels (attention.hip) hold a whole
// (atom, head) item in LDS, which bounds S by the LDS size and needs head_dim
// a multiple of 16; these stream an item's keys (forward, dQ) or queries (dK,
// dV) through LDS in tiles of KT rows, so S is unbounded, and they hold
// head_dim in a padded width HD (the next multiple of 16), loading the
// missing columns as zeros and storing only the real ones.
//
// Semantics are the reference's (peterspackman/pet-kokkos
// src/attention.cpp:205-266 forward, :1570-1697 Queries and Keys, with any
// head_dim through its generic path, :28-39, and any S through its flat
// range, :195-203). Like the reference's two backward passes, the backward is
// two kernels that each recompute the scores from the saved (max, 1/sum):
//   - the query pass: a workgroup per (atom, head, 64 queries); wave w holds
//     its 16 queries' q and dO and walks the atom's keys -> dQ;
//   - the key pass: a workgroup per (atom, head, 64 keys); wave w holds its 16
//     keys' k and v and walks the atom's queries -> dK, dV and the cf shares.
// Each output has one owner summing in a fixed order: bit-repeatable.
//
// MFMA lane layout as in attention.hip (lane l = (c, g) = (l % 16, l / 16),
// operand a = A[c][g], b = B[g][c], register r of the result = C[4g + r][c]).
// The forward and query pass form S^T = K Q^T (a lane: query c against keys
// 4g + r); the key pass forms S = Q K^T (a lane: key c against queries
// 4g + r), so its dS is already the b operand of dK^T = Q^T dS and its A that
// of dV^T = dO^T A.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <set>
#include <type_traits>
#include <utility>

#include "../../include/pet_attn.h"
#include "attn_common.h"

namespace pet_attn {

namespace {

// Column access to a head's slice when head_dim hd < HD: G 0, hd == HD (16-byte
// loads); G 1, hd a multiple of 4 (16-byte loads of whole 4-column chunks, a
// chunk past hd is zeros); G 2, any hd (4-byte loads, 4-byte alignment).
template <int W, int G>
__device__ __forceinline__ void cols_get(const float* p, int c0, int hd, float* out) {
  if constexpr (G == 0) {
    gmem_get<W>(p + c0, out);
  } else if constexpr (G == 1) {
#pragma unroll
    for (int t = 0; t < W; t += 4) {
      if (c0 + t < hd) {
        const float4 x = *reinterpret_cast<const float4*>(p + c0 + t);
        out[t] = x.x, out[t + 1] = x.y, out[t + 2] = x.z, out[t + 3] = x.w;
      } else {
        out[t] = out[t + 1] = out[t + 2] = out[t + 3] = 0.f;
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < W; ++t) out[t] = c0 + t < hd ? p[c0 + t] : 0.f;
  }
}

// W columns c0.. of head slice `col` (a column of the whole row: block offset
// plus h hd) of qkv row r, with the fused transform (row scale, bias).
template <int W, int G, bool XF>
__device__ __forceinline__ void qkv_cols(const float* qkv, int64_t ldq, size_t r, int col, int c0, int hd,
                                         const QkvXf& xf, float* out) {
  cols_get<W, G>(qkv + r * ldq + col, c0, hd, out);
  if constexpr (!XF) return;
  if (xf.rs) {
    const float sc = xf.rs[r];
#pragma unroll
    for (int t = 0; t < W; ++t) out[t] *= sc;
  }
  if (xf.b) {
    float bb[W];
    cols_get<W, G>(xf.b + col, c0, hd, bb);
#pragma unroll
    for (int t = 0; t < W; ++t) out[t] += bb[t];
  }
}

// A lane's W = HD/4 result columns c0.. (from the DT result tiles) times f,
// only the columns below hd.
template <int HD, int G>
__device__ __forceinline__ void cols_put(float* p, int c0, int hd, const f4* acc, float f) {
  constexpr int W = HD / 4, DT = HD / 16;
  if constexpr (G == 0) {
    store_slice<HD>(p + c0, acc, f);
  } else if constexpr (G == 1) {
#pragma unroll
    for (int e = 0; e < W; e += 4)
      if (c0 + e < hd)
        *reinterpret_cast<float4*>(p + c0 + e) =
            make_float4(tile_elem<DT>(acc, e) * f, tile_elem<DT>(acc, e + 1) * f, tile_elem<DT>(acc, e + 2) * f,
                        tile_elem<DT>(acc, e + 3) * f);
  } else {
#pragma unroll
    for (int e = 0; e < W; ++e)
      if (c0 + e < hd) p[c0 + e] = tile_elem<DT>(acc, e) * f;
  }
}

// Rows of a streamed tile, and the LDS of a kernel's tiles: two [KT, HD + 4]
// row blocks (pitch HD + 4: a 16-lane column of 128-bit reads touches distinct
// banks) and `extra` per-row floats; 67.6 KB at head_dim 128.
constexpr int KT = 64;
template <int HD>
constexpr size_t stream_lds_bytes(int extra) {
  return sizeof(float) * (size_t(2) * KT * (HD + 4) + size_t(extra) * KT);
}

// log cf of slot s of atom n (kOff past its count or for cf <= 0)
__device__ __forceinline__ float slot_lcf(const float* cf_seq, int64_t ldc, const Atom& at, int s) {
  if (s >= at.cnt) return kOff;
  const float cf = cf_seq[size_t(at.n) * ldc + s];
  return cf > 0.f ? log_cf(cf) : kOff;
}

// ---- forward -------------------------------------------------------------------
// Workgroup (item, query group qg): wave w owns query block 4 qg + w. Keys
// stream through LDS KT rows at a time; online softmax per 16-key block.
template <int HD, int G, bool XF>
__global__ void __launch_bounds__(256) fwd_stream_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                         const int* __restrict__ off, int N, int n0, int64_t eb,
                                                         int S, int H, int hd, float sc,
                                                         const float* __restrict__ cf_seq, int64_t ldc,
                                                         float* __restrict__ merged, int64_t ldm,
                                                         float* __restrict__ ml, QkvXf xf, int QG) {
  constexpr int W = HD / 4, DT = HD / 16, P = HD + 4, TQ = 256 / KT;
  extern __shared__ float lds[];
  float *Ks = lds, *Vs = Ks + KT * P, *lcf = Vs + KT * P;
  const int item = blockIdx.x / QG, qg = blockIdx.x - item * QG;
  const Atom at(off, item, H, N, S, n0, eb);
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int D = H * hd, hoff = at.h * hd;
  const int i = 64 * qg + 16 * w + c;  // this lane's query slot
  if (64 * qg >= at.cnt) {  // no token of this group: only the sentinel statistics
    if (ml && g == 0 && i < S) {
      float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
      mlq[0] = kOff, mlq[1] = 0.f;
    }
    return;
  }
  const bool real = i < at.cnt, active = 64 * qg + 16 * w < at.cnt;
  float q[W];
  if (real)
    qkv_cols<W, G, XF>(qkv, ldq, at.row(i), hoff, g * W, hd, xf, q);
  else
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = 0.f;
  float mx = kFloor, sum = 0.f;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  // the tile's loads: thread tid takes row tid / TQ, columns (tid % TQ) * CW ..
  constexpr int CW = HD / TQ;
  const int lr = tid / TQ, lc0 = (tid % TQ) * CW;
  for (int k0 = 0; k0 < at.cnt; k0 += KT) {
    {
      const int key = k0 + lr;
      float kv[CW], vv[CW];
      if (key < at.cnt) {
        const size_t r = at.row(key);
        qkv_cols<CW, G, XF>(qkv, ldq, r, D + hoff, lc0, hd, xf, kv);
        qkv_cols<CW, G, XF>(qkv, ldq, r, 2 * D + hoff, lc0, hd, xf, vv);
      } else {
#pragma unroll
        for (int t = 0; t < CW; ++t) kv[t] = vv[t] = 0.f;
      }
#pragma unroll
      for (int t = 0; t < CW; t += 4) {
        *reinterpret_cast<float4*>(Ks + lr * P + lc0 + t) = make_float4(kv[t], kv[t + 1], kv[t + 2], kv[t + 3]);
        *reinterpret_cast<float4*>(Vs + lr * P + lc0 + t) = make_float4(vv[t], vv[t + 1], vv[t + 2], vv[t + 3]);
      }
      if (tid % TQ == 0) lcf[lr] = slot_lcf(cf_seq, ldc, at, key);
    }
    lds_barrier();
    if (active) {
      for (int J = 0; J < KT / 16 && k0 + 16 * J < at.cnt; ++J) {
        f4 s = {0.f, 0.f, 0.f, 0.f};
        float k[W];
        lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
#pragma unroll
        for (int t = 0; t < W; ++t) s = mfma(k[t], q[t], s);
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
          for (int t = 0; t < DT; ++t) acc[t] = mfma(v[t], p[r], acc[t]);
        }
      }
    }
    lds_barrier();
  }
  const float tot = sum_g(sum);
  const bool live = real && (i == 0 || slot_lcf(cf_seq, ldc, at, i) > -1e29f);
  const float invl = live && tot > 0.f ? 1.0f / tot : 0.f;
  if (real) cols_put<HD, G>(merged + at.grow(i) * ldm + hoff, g * W, hd, acc, invl);
  if (ml && g == 0 && i < S) {
    float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    mlq[0] = live && tot > 0.f ? mx : kOff, mlq[1] = invl;
  }
}

// ---- backward: the query pass (dQ) ----------------------------------------------
template <int HD, int G, bool XF>
__global__ void __launch_bounds__(256) bwd_q_stream_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                           const int* __restrict__ off, int N, int n0, int64_t eb,
                                                           int S, int H, int hd, float sc,
                                                           const float* __restrict__ dmerged, int64_t ldg,
                                                           const float* __restrict__ merged, int64_t ldm,
                                                           const float* __restrict__ ml,
                                                           const float* __restrict__ cf_seq, int64_t ldc,
                                                           float* __restrict__ qkv_adj, int64_t lda, QkvXf xf,
                                                           int QG) {
  constexpr int W = HD / 4, DT = HD / 16, P = HD + 4, TQ = 256 / KT, CW = HD / TQ;
  extern __shared__ float lds[];
  float *Ks = lds, *Vs = Ks + KT * P, *lcf = Vs + KT * P;
  const int item = blockIdx.x / QG, qg = blockIdx.x - item * QG;
  const Atom at(off, item, H, N, S, n0, eb);
  if (64 * qg >= at.cnt) return;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int D = H * hd, hoff = at.h * hd;
  const int i = 64 * qg + 16 * w + c;
  const bool real = i < at.cnt, active = 64 * qg + 16 * w < at.cnt;
  float q[W], go[W], mi = kOff, li = 0.f, dqi = 0.f;
  if (real) {
    const size_t r = at.row(i);
    qkv_cols<W, G, XF>(qkv, ldq, r, hoff, g * W, hd, xf, q);
    cols_get<W, G>(dmerged + r * ldg + hoff, g * W, hd, go);
    float o[W];
    cols_get<W, G>(merged + at.grow(i) * ldm + hoff, g * W, hd, o);
    float d = 0.f;
#pragma unroll
    for (int t = 0; t < W; ++t) d += go[t] * o[t];
    dqi = d;
    const float* m2 = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    mi = m2[0], li = m2[1];
  } else {
#pragma unroll
    for (int t = 0; t < W; ++t) q[t] = go[t] = 0.f;
  }
  dqi = sum_g(dqi);  // Dq = dO . O of query i
  const float mie = li > 0.f ? mi : 1e30f;
  f4 dq[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = f4{0.f, 0.f, 0.f, 0.f};
  const int lr = tid / TQ, lc0 = (tid % TQ) * CW;
  for (int k0 = 0; k0 < at.cnt; k0 += KT) {
    {
      const int key = k0 + lr;
      float kv[CW], vv[CW];
      if (key < at.cnt) {
        const size_t r = at.row(key);
        qkv_cols<CW, G, XF>(qkv, ldq, r, D + hoff, lc0, hd, xf, kv);
        qkv_cols<CW, G, XF>(qkv, ldq, r, 2 * D + hoff, lc0, hd, xf, vv);
      } else {
#pragma unroll
        for (int t = 0; t < CW; ++t) kv[t] = vv[t] = 0.f;
      }
#pragma unroll
      for (int t = 0; t < CW; t += 4) {
        *reinterpret_cast<float4*>(Ks + lr * P + lc0 + t) = make_float4(kv[t], kv[t + 1], kv[t + 2], kv[t + 3]);
        *reinterpret_cast<float4*>(Vs + lr * P + lc0 + t) = make_float4(vv[t], vv[t + 1], vv[t + 2], vv[t + 3]);
      }
      if (tid % TQ == 0) lcf[lr] = slot_lcf(cf_seq, ldc, at, key);
    }
    lds_barrier();
    if (active) {
      for (int J = 0; J < KT / 16 && k0 + 16 * J < at.cnt; ++J) {
        f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
        {
          float k[W], v[W];
          lds_get<W>(Ks + (16 * J + c) * P + g * W, k);
          lds_get<W>(Vs + (16 * J + c) * P + g * W, v);
#pragma unroll
          for (int t = 0; t < W; ++t) st = mfma(k[t], q[t], st), dp = mfma(v[t], go[t], dp);
        }
        float lc[4], ds[4];
        lds_get<4>(lcf + 16 * J + 4 * g, lc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // query i, key k0 + 16 J + 4 g + r
          const float a = __expf(st[r] * sc + lc[r] - mie) * li;
          ds[r] = a * (dp[r] - dqi);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float kk[DT];
          lds_get<DT>(Ks + (16 * J + 4 * g + r) * P + c * DT, kk);
#pragma unroll
          for (int t = 0; t < DT; ++t) dq[t] = mfma(kk[t], ds[r], dq[t]);
        }
      }
    }
    lds_barrier();
  }
  if (real) cols_put<HD, G>(qkv_adj + at.row(i) * lda + hoff, g * W, hd, dq, sc);
}

// ---- backward: the key pass (dK, dV, cf shares) -----------------------------------
template <int HD, int G, bool XF>
__global__ void __launch_bounds__(256) bwd_kv_stream_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                            const int* __restrict__ off, int N, int n0, int64_t eb,
                                                            int S, int H, int hd, float sc,
                                                            const float* __restrict__ dmerged, int64_t ldg,
                                                            const float* __restrict__ merged, int64_t ldm,
                                                            const float* __restrict__ ml,
                                                            const float* __restrict__ cf_seq, int64_t ldc,
                                                            float* __restrict__ qkv_adj, int64_t lda,
                                                            float* __restrict__ cfh, QkvXf xf, int KG) {
  constexpr int W = HD / 4, DT = HD / 16, P = HD + 4, QT = KT, TQ = 256 / QT, CW = HD / TQ;
  extern __shared__ float lds[];
  float *Qs = lds, *Gs = Qs + QT * P, *mis = Gs + QT * P, *lis = mis + QT, *dqs = lis + QT;
  const int item = blockIdx.x / KG, kg = blockIdx.x - item * KG;
  const Atom at(off, item, H, N, S, n0, eb);
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, c = l & 15, g = l >> 4;
  const int k = 64 * kg + 16 * w + c;  // this lane's key slot
  float* cfrow = cfh + (size_t(at.n) * H + at.h) * S;
  if (64 * kg >= at.cnt) {  // no token of this group: zero cf shares
    if (g == 0 && k < S) cfrow[k] = 0.f;
    return;
  }
  const int D = H * hd, hoff = at.h * hd;
  const bool real = k < at.cnt, active = 64 * kg + 16 * w < at.cnt;
  float kr[W], vr[W];
  if (real) {
    const size_t r = at.row(k);
    qkv_cols<W, G, XF>(qkv, ldq, r, D + hoff, g * W, hd, xf, kr);
    qkv_cols<W, G, XF>(qkv, ldq, r, 2 * D + hoff, g * W, hd, xf, vr);
  } else {
#pragma unroll
    for (int t = 0; t < W; ++t) kr[t] = vr[t] = 0.f;
  }
  const float lck = slot_lcf(cf_seq, ldc, at, k);
  f4 dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  const int lr = tid / TQ, lc0 = (tid % TQ) * CW;
  for (int i0 = 0; i0 < at.cnt; i0 += QT) {
    {
      const int qi = i0 + lr;
      float qv[CW], gv[CW], d = 0.f, mi = 0.f, li = 0.f;
      if (qi < at.cnt) {
        const size_t r = at.row(qi);
        qkv_cols<CW, G, XF>(qkv, ldq, r, hoff, lc0, hd, xf, qv);
        cols_get<CW, G>(dmerged + r * ldg + hoff, lc0, hd, gv);
        float o[CW];
        cols_get<CW, G>(merged + at.grow(qi) * ldm + hoff, lc0, hd, o);
#pragma unroll
        for (int t = 0; t < CW; ++t) d += gv[t] * o[t];
        const float* m2 = ml + 2 * ((size_t(at.n) * H + at.h) * S + qi);
        mi = m2[0], li = m2[1];
      } else {
#pragma unroll
        for (int t = 0; t < CW; ++t) qv[t] = gv[t] = 0.f;
      }
      // Dq of the row over its TQ column shares (consecutive lanes)
#pragma unroll
      for (int m = 1; m < TQ; m <<= 1) d += __shfl_xor(d, m);
#pragma unroll
      for (int t = 0; t < CW; t += 4) {
        *reinterpret_cast<float4*>(Qs + lr * P + lc0 + t) = make_float4(qv[t], qv[t + 1], qv[t + 2], qv[t + 3]);
        *reinterpret_cast<float4*>(Gs + lr * P + lc0 + t) = make_float4(gv[t], gv[t + 1], gv[t + 2], gv[t + 3]);
      }
      if (tid % TQ == 0) {
        mis[lr] = li > 0.f ? mi : 1e30f;  // a query with no live key: exp underflows to 0
        lis[lr] = li;
        dqs[lr] = d;
      }
    }
    lds_barrier();
    if (active) {
      for (int I = 0; I < QT / 16 && i0 + 16 * I < at.cnt; ++I) {
        f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
        {
          float qa[W], ga[W];
          lds_get<W>(Qs + (16 * I + c) * P + g * W, qa);
          lds_get<W>(Gs + (16 * I + c) * P + g * W, ga);
#pragma unroll
          for (int t = 0; t < W; ++t) st = mfma(qa[t], kr[t], st), dp = mfma(ga[t], vr[t], dp);
        }
        float a[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // query i0 + 16 I + 4 g + r, key k
          const int qr = 16 * I + 4 * g + r;
          a[r] = __expf(st[r] * sc + lck - mis[qr]) * lis[qr];
          ds[r] = a[r] * (dp[r] - dqs[qr]);
          cfa += ds[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float qq[DT], gg[DT];
          lds_get<DT>(Qs + (16 * I + 4 * g + r) * P + c * DT, qq);
          lds_get<DT>(Gs + (16 * I + 4 * g + r) * P + c * DT, gg);
#pragma unroll
          for (int t = 0; t < DT; ++t) dk[t] = mfma(qq[t], ds[r], dk[t]), dv[t] = mfma(gg[t], a[r], dv[t]);
        }
      }
    }
    lds_barrier();
  }
  const float cft = sum_g(cfa);
  if (real) {
    float* o = qkv_adj + at.row(k) * lda + hoff;
    cols_put<HD, G>(o + D, g * W, hd, dk, sc);
    cols_put<HD, G>(o + 2 * D, g * W, hd, dv, 1.0f);
  }
  if (g == 0 && k < S) cfrow[k] = real ? cft : 0.f;
}

template <class F>
int with_padded_head_dim(int hd, F&& f) {
  switch ((hd + 15) / 16) {
    case 1: return f(std::integral_constant<int, 16>{});
    case 2: return f(std::integral_constant<int, 32>{});
    case 3: return f(std::integral_constant<int, 48>{});
    case 4: return f(std::integral_constant<int, 64>{});
    case 5: return f(std::integral_constant<int, 80>{});
    case 6: return f(std::integral_constant<int, 96>{});
    case 7: return f(std::integral_constant<int, 112>{});
    case 8: return f(std::integral_constant<int, 128>{});
    default: return PET_ATTN_EHEADDIM;
  }
}

// Lets kernel k take `bytes` of dynamic LDS (above the 64 KB default), once
// per device.
template <class K>
bool raise_lds(K k, size_t bytes) {
  if (bytes <= 65536) return true;
  static std::mutex mu;
  static std::set<std::pair<int, const void*>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const void* kp = reinterpret_cast<const void*>(k);
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({dev, kp})) return true;
  if (hipFuncSetAttribute(kp, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) != hipSuccess) return false;
  done.insert({dev, kp});
  return true;
}

// G of a head_dim (see cols_get)
int column_mode(int hd) { return hd % 16 == 0 ? 0 : hd % 4 == 0 ? 1 : 2; }

template <class F>
int with_modes(int hd, bool xf, F&& f) {
  return with_padded_head_dim(hd, [&](auto hdc) {
    switch (column_mode(hd)) {
      case 0: return xf ? f(hdc, std::integral_constant<int, 0>{}, std::true_type{})
                        : f(hdc, std::integral_constant<int, 0>{}, std::false_type{});
      case 1: return xf ? f(hdc, std::integral_constant<int, 1>{}, std::true_type{})
                        : f(hdc, std::integral_constant<int, 1>{}, std::false_type{});
      default: return xf ? f(hdc, std::integral_constant<int, 2>{}, std::true_type{})
                         : f(hdc, std::integral_constant<int, 2>{}, std::false_type{});
    }
  });
}

}  // namespace

int stream_fwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, hipStream_t st) {
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  const int QG = (sh.slots + 63) / 64;
  if (items * QG >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  return with_modes(sh.head_dim, xf.rs || xf.b, [&](auto hdc, auto gc, auto xc) {
    constexpr int HD = decltype(hdc)::value, G = decltype(gc)::value;
    constexpr bool XF = decltype(xc)::value;
    auto kern = fwd_stream_kernel<HD, G, XF>;
    const size_t bytes = stream_lds_bytes<HD>(1);
    if (!raise_lds(kern, bytes)) return PET_ATTN_ELAUNCH;
    hipLaunchKernelGGL(kern, dim3(unsigned(items * QG)), dim3(256), bytes, st, qkv, ldq, off,
                       sh.n_atoms, n0, eb, sh.slots, sh.heads, sh.head_dim, sh.scale, cf_seq, ldc, merged, ldm, ml, xf,
                       QG);
    return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
  });
}

int stream_bwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
               const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
               const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, hipStream_t st) {
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  const int QG = (sh.slots + 63) / 64;
  if (items * QG >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  return with_modes(sh.head_dim, xf.rs || xf.b, [&](auto hdc, auto gc, auto xc) {
    constexpr int HD = decltype(hdc)::value, G = decltype(gc)::value;
    constexpr bool XF = decltype(xc)::value;
    auto kq = bwd_q_stream_kernel<HD, G, XF>;
    auto kkv = bwd_kv_stream_kernel<HD, G, XF>;
    const size_t bq = stream_lds_bytes<HD>(1), bkv = stream_lds_bytes<HD>(3);
    if (!raise_lds(kq, bq) || !raise_lds(kkv, bkv)) return PET_ATTN_ELAUNCH;
    hipLaunchKernelGGL(kq, dim3(unsigned(items * QG)), dim3(256), bq, st, qkv, ldq, off,
                       sh.n_atoms, n0, eb, sh.slots, sh.heads, sh.head_dim, sh.scale, dmerged, ldg, merged, ldm, ml,
                       cf_seq, ldc, qkv_adj, lda, xf, QG);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
    hipLaunchKernelGGL(kkv, dim3(unsigned(items * QG)), dim3(256), bkv, st, qkv, ldq,
                       off, sh.n_atoms, n0, eb, sh.slots, sh.heads, sh.head_dim, sh.scale, dmerged, ldg, merged, ldm,
                       ml, cf_seq, ldc, qkv_adj, lda, cfh, xf, QG);
    return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
  });
}

}  // namespace pet_attn
