// The attention backward at head_dim 32 from fp16 pairs on gfx950's 16-bit
// matrix cores: every product of the backward (S, dP, dK, dV, dQ) at fp32
// accuracy in three f16 matrix instructions where the fp32 instruction takes
// eight (split_bf16.h: an fp32 x scaled by a power of two splits into an fp16
// hi holding its leading 11 bits and an fp16 lo holding the next 11).
//
// Semantics: the reference's attention_bwd core (peterspackman/pet-kokkos
// src/attention.cpp:1570-1697, Queries<HD> and Keys<HD,DK,DV>, and its MFMA
// backward :451-593): for query i and key j of an (atom, head),
//   P_ij = exp(sc q_i.k_j + log cf_j - m_i) / l_i   (m, 1/l the forward's ml)
//   dS_ij = P_ij (dO_i.v_j - dO_i.O_i)
//   dQ_i = sc sum_j dS_ij k_j, dK_j = sc sum_i dS_ij q_i, dV_j = sum_i P_ij dO_i,
//   cfh_j = sum_i dS_ij (the cf adjoint's share of this head).
//
// Work decomposition: one workgroup per (atom, head), wave w owning key block
// w (16 keys). At step s wave w takes query block I = (w + s) mod nb:
//   S = Q_I K_w^T and dP = dO_I V_w^T on the 16x16x32 instruction, a lane
//   holding key 16w + c against queries 16I + 4g + r (lane l = (c, g) =
//   (l % 16, l / 16), register r of the result);
//   P and dS, scaled and split in registers, are then already the b operand
//   of the 16x16x16 instruction for dV_w^T += dO_I^T P and dK_w^T += Q_I^T dS
//   (k = the block's 16 queries), so the key block's dK and dV never leave the
//   wave's registers; only dS goes through LDS to the owner of query block
//   I, which adds dQ_I^T += K_w^T dS^T after the step's barrier.
// Every product is formed once, every output has one owner summing in a fixed
// order, nothing is atomic: results repeat bit for bit.
//
// Scales: per item, powers of two put the largest |Q|, |K|, |V|, |dO| at
// [2^14, 2^15) (so everything down to 2^-29 of the item's largest value keeps
// 22 significand bits), P is scaled by 2^15 (P <= 1), and dS by the power of
// two that puts the bound max|v| max|dO| + max|dO.O| >= max|dS| there (row
// norms).
// The scales are undone in fp32 where the results are stored.
//
// LDS (R = 16 NW rows): Q, dO, K as hi and lo planes, token-major (a lane's
// 8 dims one 16-byte store; Q's and dO's rows for S and dP read straight, the
// a operand of dK, dV and dQ -- a dim's four consecutive tokens -- through the
// transposing read; rows padded at head_dim 32, unpadded with permuted chunks
// at 64: tok_off), the per-query (max, 2^15 / sum, scaled dO.O), and two
// buffers of one dS tile a wave (hi and lo, [16 keys][16 queries + 4 pad]).
// 51.1 KB at 5 waves and head_dim 32 (three workgroups a CU), 75.4 KB at 64
// (two).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "../../include/pet_attn.h"
#include "attn_common.h"
#include "split_bf16.h"

// No implicit contraction in this file: a split's hi and lo must come from one
// rounded fp32 value, and a multiply contracted into lo's subtraction (an
// fma_mix on the unrounded product) can disagree with the hi taken from the
// rounded product by an fp16 ulp. Where a fused multiply-add is meant, fmaf.
#pragma clang fp contract(off)

namespace pet_attn {

using pet_split::mfma3;
using pet_split::mfma3_16;
using pet_split::mfma4;
using pet_split::mfma4_16;
using pet_split::u2;
using pet_split::u4;

namespace {

constexpr int kPairHD = 32;
constexpr int kPairMaxWaves = 8;  // 128 slots; beyond, the tile-exchange kernel

struct PairLds {
  static constexpr int TP = 20;  // halves a dS tile row (16 queries, 4 of pad)
  static constexpr int TS = 16 * TP;  // halves a tile part
  // The planes token-major (a token's dims a row, tok_off: a lane's 8 dims
  // one 16-byte store), rows padded at head_dim 32
  static constexpr bool pad(int HD) { return HD <= 32; }
  int R, PT;  // rows; plane pitch in halves
  size_t pl, st, red, tb, bytes;
  __host__ __device__ constexpr PairLds(int HD, int NW)
      : R(16 * NW), PT(pad(HD) ? HD + 8 : HD), pl(0),
        st(pl + size_t(6) * 16 * NW * PT * 2),  // 6 planes: Q, dO, K, each hi then lo
        red(st + size_t(3) * R * 4),            // 8 words a wave: its maxima
        tb(red + size_t(8) * NW * 4), bytes(tb + size_t(2) * NW * 2 * TS * 2) {}
};

// gfx950's transposing LDS read (ds_read_b64_tr_b16), on the 16 lanes of a
// row: lane j's element m is element j % 4 of what lane 4m + j / 4 addressed.
// A lane addressing the four consecutive tokens 4(L % 4) .. + 3 of plane row
// d0 + L / 4 thus receives its own token's dims d0 .. d0 + 3.
typedef short s4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u2 lds_tr16(const _Float16* p) {
  typedef __attribute__((address_space(3))) s4 lds_s4;
  return __builtin_bit_cast(u2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p)));
}

// Token-major planes of HD dims: the offset in halves of row r's 16-byte
// chunk ch (8 dims). Padded (PAD): rows of HD + 8 halves, the 16 rows a
// 16-byte read meets on distinct banks. Unpadded, where LDS allows no pad (the
// backward at head_dim 64, two workgroups a CU): rows of HD halves with each
// row's chunks permuted by an XOR of bits of the row, found by a search for
// conflict-free 16-byte and transposing reads. Measured on MI355X: the padded
// rows faster at head_dim 32 (C3 backward 242 against 251 us with the
// permutation) and in the forward at 64 (C5 840 against 850 us); the
// unpadded rows take the head_dim-64 backward from dim-major planes 2470 to
// 2227 us (C5).
template <int HD, bool PAD>
__device__ __forceinline__ int tok_off(int r, int ch) {
  static_assert(HD == 32 || HD == 64, "head_dim 32 or 64");
  if constexpr (PAD) {
    return r * (HD + 8) + 8 * ch;
  } else {
    const int b1 = (r >> 1) & 1, b2 = (r >> 2) & 1, b3 = (r >> 3) & 1;
    const int h = HD == 32 ? (b2 << 1) ^ b3 : (b1 << 1) ^ (b2 << 2) ^ b3;
    return r * HD + 8 * (ch ^ h);
  }
}

// An opaque 1.0 in a register (an empty asm, no instruction): fmaf(x, one, -h)
// then cannot fold into a subtraction, so the remainder of a split is one
// v_fma_mix reading the fp16 h directly, not a conversion back to fp32 and a
// subtraction.
__device__ __forceinline__ float opaque_one() {
  float o = 1.f;
  asm("" : "+v"(o));
  return o;
}
// Two values as fp16 (hi, lo) registers, both to nearest: hi the fp16 nearest
// x, lo the fp16 nearest x - hi (exact in fp32): |x - hi - lo| <= 2^-23 |x|,
// or <= 2^-25 below fp16's normal range (|x| < 2^15 here). x and y are pinned
// to registers first (an empty asm), so both parts come from one rounded fp32
// value: a multiply fused into the fp16 conversion (fma_mix on the unrounded
// product) could otherwise give hi and lo different x's. Three instructions
// for two values: one packed conversion, two fma_mix.
__device__ __forceinline__ void pair2x(float x, float y, float one, unsigned& hi, unsigned& lo) {
  asm("" : "+v"(x), "+v"(y));
  const pet_split::h2v h = {(_Float16)x, (_Float16)y};
  const pet_split::h2v l = {(_Float16)fmaf(x, one, -float(h[0])), (_Float16)fmaf(y, one, -float(h[1]))};
  hi = __builtin_bit_cast(unsigned, h);
  lo = __builtin_bit_cast(unsigned, l);
}
// pair2x of x s and y s for a power of two s (exact products): hi and the
// remainder x s - hi are each one fma_mix from x and s (hi's an fma with 0,
// which the compiler cannot turn back into a multiply: it differs from x s
// only in the sign of a zero), four instructions for the two values.
__device__ __forceinline__ void pair2s(float x, float y, float s, unsigned& hi, unsigned& lo) {
  const pet_split::h2v h = {(_Float16)fmaf(x, s, 0.f), (_Float16)fmaf(y, s, 0.f)};
  const pet_split::h2v l = {(_Float16)fmaf(x, s, -float(h[0])), (_Float16)fmaf(y, s, -float(h[1]))};
  hi = __builtin_bit_cast(unsigned, h);
  lo = __builtin_bit_cast(unsigned, l);
}

// The largest x over a row of 16 lanes, in every lane of the row, for x >= 0
// (norms): DPP row rotations by 1, 2, 4, 8, each folded into an integer max
// of the bit patterns (which order non-negative floats as their values do;
// fmaxf would canonicalize each operand first, an instruction more a step).
// A rotation within a full row reads a live lane everywhere, so the DPP's old
// value (0) is never taken.
__device__ __forceinline__ float row_max16(float x) {
  int v = __float_as_int(x);
#define PET_ROR(n) v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x120 + (n), 0xf, 0xf, true))
  PET_ROR(1);
  PET_ROR(2);
  PET_ROR(4);
  PET_ROR(8);
#undef PET_ROR
  return __int_as_float(v);
}
// The exponent k of the pair scale 2^k that puts m = f 2^e (f in [0.5, 1))
// at [2^14, 2^15): 15 - e; 0 for a zero (or non-finite) m.
__device__ __forceinline__ int pair_exp(float m) {
  if (!(m > 0.f) || m > 3.0e38f) return 0;
  return min(15 - __builtin_amdgcn_frexp_expf(m), 126);
}

// The fused QKV transform (QkvXf: qkv[r][j] rs[r] + b[j]) applied to a lane's
// q, k, v values (dims col0 + 32kc .. + 7 of each) once every row load of
// the item is issued: the row scale loaded once, the bias per chunk.
template <int KC>
__device__ __forceinline__ void xf_rows(const QkvXf& xf, size_t r, int col0, int D, float* q, float* k, float* v) {
  const float sr = xf.rs ? xf.rs[r] : 1.f;
  float* x[3] = {q, k, v};
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      float bb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (xf.b) gmem_get<8>(xf.b + m * D + col0 + 32 * kc, bb);
#pragma unroll
      for (int t = 0; t < 8; ++t) x[m][8 * kc + t] = fmaf(x[m][8 * kc + t], sr, bb[t]);
    }
}
// qkv_get with the transform but no branch: a missing row scale or bias reads
// a valid address (the row itself) and selects 1 or 0, so one chunk's loads
// and the next chunk's stay in one block and are all in flight together.
template <bool XF>
__device__ __forceinline__ void qkv_get8(const float* qkv, int64_t ldq, size_t r, int col, const QkvXf& xf,
                                         float* out) {
  const float* row = qkv + r * ldq + col;
  gmem_get<8>(row, out);
  if constexpr (!XF) return;
  const bool hs = xf.rs != nullptr, hb = xf.b != nullptr;
  const float s0 = *(hs ? xf.rs + r : row);
  float bb[8];
  gmem_get<8>(hb ? xf.b + col : row, bb);
  const float sr = hs ? s0 : 1.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) out[t] = fmaf(out[t], sr, hb ? bb[t] : 0.f);
}
}  // namespace

// The backward's arguments (one launch).
struct PairBwdArgs {
  const float* qkv;
  int64_t ldq;
  const int* off;
  int N, n0;
  int64_t eb;
  int S, H;
  float sc;
  const float* dmerged;
  int64_t ldg;
  const float* merged;
  int64_t ldm;
  const float* ml;
  const float* cf_seq;
  int64_t ldc;
  float* qkv_adj;
  int64_t lda;
  float* cfh;
  QkvXf xf;
  // block pairs in place of qkv_adj (kernel form BP): the rows of qkv_adj as
  // fp16 pairs (8-value groups of hi then lo 16 bytes, 3D / 8 groups a row),
  // each (row, head, q | k | v) slice of HD values scaled by its own power of
  // two, then the slices' inverse scales [3H][prows] (block m H + h)
  u4* qpairs = nullptr;
  int64_t prows = 0;
};

// A lane's raw rows of one item: its slot's q, k, v, dO and O (dims 32kc + 8g
// .. + 7) and the slot's saved statistics and cf as loaded (slot 0's past the
// count: the item masks them where it reads them, so that nothing waits on
// the loads when they are issued).
template <int W>
struct PairRows {
  float q[W], k[W], v[W], go[W], oo[W];
  float mi, li, pcf;
};

// Issues the loads of a lane's rows of item `at` (wave w, lane (c, g), slot i =
// 16 w + c). A slot past the count loads slot 0's rows instead of zeros: as a
// query it has 1/sum 0 and as a key log cf kOff, so its P and dS are exactly 0
// and it adds nothing (and, a copy of a row of the item, it moves no scale).
template <int HD, bool XF>
__device__ __forceinline__ void pair_bwd_load(const PairBwdArgs& a, const Atom& at, int w, int g, int i,
                                              PairRows<HD / 4>& r) {
  constexpr int KC = HD / 32;
  constexpr bool XF_LATE = XF && KC == 1;
  const int D = a.H * HD;
  const bool active = w < at.nb, real = active && i < at.cnt;
  r.mi = kOff, r.li = 0.f, r.pcf = 0.f;  // an idle wave's
  if (active) {  // wave-uniform
    const int si = real ? i : 0;
    const size_t row = at.row(si);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int col = at.h * HD + 32 * kc + 8 * g;
      if constexpr (XF_LATE) {
        gmem_get<8>(a.qkv + row * a.ldq + col, r.q + 8 * kc);
        gmem_get<8>(a.qkv + row * a.ldq + D + col, r.k + 8 * kc);
        gmem_get<8>(a.qkv + row * a.ldq + 2 * D + col, r.v + 8 * kc);
      } else {
        qkv_get8<XF>(a.qkv, a.ldq, row, col, a.xf, r.q + 8 * kc);
        qkv_get8<XF>(a.qkv, a.ldq, row, D + col, a.xf, r.k + 8 * kc);
        qkv_get8<XF>(a.qkv, a.ldq, row, 2 * D + col, a.xf, r.v + 8 * kc);
      }
      gmem_get<8>(a.dmerged + row * a.ldg + col, r.go + 8 * kc);
      gmem_get<8>(a.merged + at.grow(si) * a.ldm + col, r.oo + 8 * kc);
    }
    if constexpr (XF_LATE) xf_rows<KC>(a.xf, row, at.h * HD + 8 * g, D, r.q, r.k, r.v);
    const float* m2 = a.ml + 2 * ((size_t(at.n) * a.H + at.h) * a.S + si);
    r.mi = m2[0], r.li = m2[1], r.pcf = a.cf_seq[size_t(at.n) * a.ldc + si];
  }
}

// One (atom, head) item of the backward from the lane's loaded rows r.
template <int HD, int NW, bool XF, bool BP = false>
__device__ __forceinline__ void pair_bwd_item(const PairBwdArgs& a, const Atom& at, PairRows<HD / 4>& r,
                                              unsigned char* lds) {
  // KC 32-dim chunks of the head: lane (c, g) holds dims 32kc + 8g .. + 7 of its row
  constexpr int KC = HD / 32, W = 8 * KC, DT = HD / 16;
  static_assert(HD % 32 == 0, "head_dim a multiple of 32");
  // the fused transform after every row load is issued (one chunk a lane at
  // head_dim 32); at 64 the raw rows held together would spill, so each
  // chunk is transformed as it arrives, branch-free (qkv_get8) so that every
  // chunk's loads are still issued together
  constexpr bool XF_LATE = XF && KC == 1;
  const int D = a.H * HD, H = a.H;
  const float sc = a.sc;
  constexpr PairLds L(HD, NW);
  constexpr int PT = L.PT, TP = PairLds::TP, TS = PairLds::TS;
  _Float16* planes = reinterpret_cast<_Float16*>(lds + L.pl);
  constexpr int PS = L.R * PT;  // halves a plane part
  constexpr bool PAD = PairLds::pad(HD);
  _Float16* QTh = planes;
  _Float16* GTh = planes + 2 * PS;
  _Float16* KTh = planes + 4 * PS;
  float* STm = reinterpret_cast<float*>(lds + L.st);
  float* STl = STm + L.R;
  float* STd = STl + L.R;
  float* red = reinterpret_cast<float*>(lds + L.red);
  _Float16* TB = reinterpret_cast<_Float16*>(lds + L.tb);

  // the wave index in a scalar register: the step's block offsets are then
  // scalar too
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;  // this lane's row: its query slot, and its key slot
  const bool active = w < at.nb, real = active && i < at.cnt;

  // ---- the wave's own block: rows 16w .. 16w + 15, lane (c, g) dims 32kc + 8g .. + 7
  float* q = r.q;
  float* k = r.k;
  float* v = r.v;
  float* go = r.go;
  float* oo = r.oo;
  const float mi = real ? r.mi : kOff, li = real ? r.li : 0.f, pcf = real ? r.pcf : 0.f;
  // Row norms (over the head's dims; every lane of a row gets its row's), then
  // their largest over the item: the scales come from them (a row's largest
  // |x| is at most its norm).
  float nq = 0.f, nk = 0.f, nv = 0.f, ng = 0.f, dot = 0.f;
#pragma unroll
  for (int t = 0; t < W; ++t) {
    nq = fmaf(q[t], q[t], nq), nk = fmaf(k[t], k[t], nk), nv = fmaf(v[t], v[t], nv), ng = fmaf(go[t], go[t], ng);
    dot = fmaf(go[t], oo[t], dot);
  }
  const float Di = sum_g(dot);  // dO_i . O_i
  float m5[5] = {sum_g(nq), sum_g(nk), sum_g(nv), sum_g(ng), Di * Di};
#pragma unroll
  for (int u = 0; u < 5; ++u) m5[u] = active ? row_max16(m5[u]) : 0.f;  // an idle wave's registers hold nothing
  if (l == 0) {
    *reinterpret_cast<float4*>(red + 8 * w) = make_float4(m5[0], m5[1], m5[2], m5[3]);
    red[8 * w + 4] = m5[4];
  }
  lds_barrier();
  float M[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int x = 0; x < NW; ++x) {
    const float4 a = *reinterpret_cast<const float4*>(red + 8 * x);
    M[0] = fmaxf(M[0], a.x), M[1] = fmaxf(M[1], a.y), M[2] = fmaxf(M[2], a.z), M[3] = fmaxf(M[3], a.w);
    M[4] = fmaxf(M[4], red[8 * x + 4]);
  }
#pragma unroll
  for (int u = 0; u < 5; ++u) M[u] = __builtin_amdgcn_sqrtf(M[u]);  // largest norms, largest |D| (only their exponents matter)
  // scales 2^k: Q, K, V, dO by their largest row norm; dS by its bound
  // |dS_ij| = P_ij |dO_i.v_j - D_i| <= max|v| max|dO| + max|D| (Cauchy-Schwarz, P <= 1)
  const int kQ = pair_exp(M[0]), kK = pair_exp(M[1]), kV = pair_exp(M[2]), kG = pair_exp(M[3]);
  const int kS = pair_exp(fmaf(M[2], M[3], M[4]));
  constexpr int kP = 15;  // P's scale 2^15
  const float sQ = __builtin_amdgcn_ldexpf(1.f, kQ), sK = __builtin_amdgcn_ldexpf(1.f, kK);
  const float sV = __builtin_amdgcn_ldexpf(1.f, kV), sG = __builtin_amdgcn_ldexpf(1.f, kG);
  const float scS = __builtin_amdgcn_ldexpf(sc, -kQ - kK);        // scores from the scaled product
  const float alpha = __builtin_amdgcn_ldexpf(1.f, kS - kP - kV - kG);  // dP's scale into dS's, over P's

  // own rows split: K and V stay in registers (the b operand of S and dP);
  // Q, dO and K go to the transposed planes
  u4 kb[KC][2], vb[KC][2];
  {
    u4 qs[KC][2], gs[KC][2];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int x = 8 * kc + 2 * j;
        unsigned h[4], lo[4];
        pair2s(q[x], q[x + 1], sQ, h[0], lo[0]);
        pair2s(go[x], go[x + 1], sG, h[1], lo[1]);
        pair2s(k[x], k[x + 1], sK, h[2], lo[2]);
        pair2s(v[x], v[x + 1], sV, h[3], lo[3]);
        qs[kc][0][j] = h[0], qs[kc][1][j] = lo[0], gs[kc][0][j] = h[1], gs[kc][1][j] = lo[1];
        kb[kc][0][j] = h[2], kb[kc][1][j] = lo[2], vb[kc][0][j] = h[3], vb[kc][1][j] = lo[3];
      }
    if (active) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {  // the lane's 8 dims of each plane, one 16-byte store
        const int o = tok_off<HD, PAD>(i, 4 * kc + g);
        *reinterpret_cast<u4*>(QTh + o) = qs[kc][0], *reinterpret_cast<u4*>(QTh + PS + o) = qs[kc][1];
        *reinterpret_cast<u4*>(GTh + o) = gs[kc][0], *reinterpret_cast<u4*>(GTh + PS + o) = gs[kc][1];
        *reinterpret_cast<u4*>(KTh + o) = kb[kc][0], *reinterpret_cast<u4*>(KTh + PS + o) = kb[kc][1];
      }
    }
    if (active) {
      if (g == 0) {
        // a query with no live key (li = 0): an exponent near -1e30, exp gives 0
        STm[i] = li > 0.f ? mi : 1e30f;
        STl[i] = __builtin_amdgcn_ldexpf(li, kP);
        STd[i] = __builtin_amdgcn_ldexpf(Di, kS - kP);
      }
    }
  }
  const float lcj = pcf > 0.f ? log_cf(pcf) : kOff;  // this lane's key's log cf (kOff past the count)

  f4 dq[DT], dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) dq[t] = dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  float cfa = 0.f;
  const int nb = at.nb;
  const float one = opaque_one();

  // Phase 1 of step s: query block I = (w + s) mod nb against the own keys.
  auto phase1 = [&](int s) {
    int I = w + s;
    if (I >= nb) I -= nb;
    // a operand: query 16I + c, dims 32kc + 8g .. + 7, read transposed from
    // the planes (rows 32kc + 8g + 4u + c / 4, tokens 16I + 4 (c % 4) .. + 3)
    f4 st = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};  // S: key 16w + c (column), queries 16I + 4g + r
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      // query 16I + c's row: its dims 32kc + 8g .. + 7 read straight
      const int o = tok_off<HD, PAD>(16 * I + c, 4 * kc + g);
      const u4 qa[2] = {*reinterpret_cast<const u4*>(QTh + o), *reinterpret_cast<const u4*>(QTh + PS + o)};
      const u4 ga[2] = {*reinterpret_cast<const u4*>(GTh + o), *reinterpret_cast<const u4*>(GTh + PS + o)};
      st = mfma3(qa, kb[kc], st);
      dp = mfma3(ga, vb[kc], dp);
    }
    const float4 m4 = *reinterpret_cast<const float4*>(STm + 16 * I + 4 * g);
    const float4 l4 = *reinterpret_cast<const float4*>(STl + 16 * I + 4 * g);
    const float4 d4 = *reinterpret_cast<const float4*>(STd + 16 * I + 4 * g);
    const float mm[4] = {m4.x, m4.y, m4.z, m4.w}, ll[4] = {l4.x, l4.y, l4.z, l4.w}, dd[4] = {d4.x, d4.y, d4.z, d4.w};
    float pp[4], ds[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pp[r] = __expf(fmaf(st[r], scS, lcj - mm[r])) * ll[r];  // 2^15 P
      ds[r] = pp[r] * fmaf(dp[r], alpha, -dd[r]);           // sS dS
      cfa += ds[r];
    }
    unsigned h[4], lo[4];
    pair2x(pp[0], pp[1], one, h[0], lo[0]);
    pair2x(pp[2], pp[3], one, h[1], lo[1]);
    pair2x(ds[0], ds[1], one, h[2], lo[2]);
    pair2x(ds[2], ds[3], one, h[3], lo[3]);
    const u2 ph = {h[0], h[1]}, pl = {lo[0], lo[1]}, sh = {h[2], h[3]}, sl = {lo[2], lo[3]};
    // dV^T += dO_I^T P and dK^T += Q_I^T dS: a operand rows 16t + c of the
    // planes, the block's queries 16I + 4g .. + 3
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      // dim 16t + c of queries 16I + 4g .. + 3, read transposed (lane 4m + q:
      // query 16I + 4g + m, dims 16t + 4q .. + 3)
      const int o = tok_off<HD, PAD>(16 * I + 4 * g + (c >> 2), 2 * t + ((c & 3) >> 1)) + 4 * (c & 1);
      const u2 gth = lds_tr16(GTh + o), gtl = lds_tr16(GTh + PS + o), qth = lds_tr16(QTh + o),
               qtl = lds_tr16(QTh + PS + o);
      dv[t] = mfma3_16(gth, gtl, ph, pl, dv[t]);
      dk[t] = mfma3_16(qth, qtl, sh, sl, dk[t]);
    }
    // dS to query block I's owner: hi and lo tiles T[key c][query 4g + r],
    // read back transposed
    _Float16* tb = TB + ((s & 1) * NW + w) * (2 * TS) + c * TP + 4 * g;
    *reinterpret_cast<u2*>(tb) = sh;
    *reinterpret_cast<u2*>(tb + TS) = sl;
  };
  // Phase 2 of step s: the own query block's tile from key block J = (w - s)
  // mod nb: dQ_w^T += K_J^T dS^T.
  auto phase2 = [&](int s) {
    int J = w - s;
    if (J < 0) J += nb;
    // b operand: query c, keys 4g .. 4g + 3 (tile rows 4g + c / 4, queries
    // 4 (c % 4) .. + 3)
    const _Float16* tb = TB + ((s & 1) * NW + J) * (2 * TS) + (4 * g + (c >> 2)) * TP + 4 * (c & 3);
    const u2 bh = lds_tr16(tb), bl = lds_tr16(tb + TS);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      // dim 16t + c of keys 16J + 4g .. + 3, read transposed
      const int o = tok_off<HD, PAD>(16 * J + 4 * g + (c >> 2), 2 * t + ((c & 3) >> 1)) + 4 * (c & 1);
      const u2 kth = lds_tr16(KTh + o), ktl = lds_tr16(KTh + PS + o);
      dq[t] = mfma3_16(kth, ktl, bh, bl, dq[t]);
    }
  };
  // Software-pipelined: between two barriers a wave has phase 2 of the last
  // step and phase 1 of this one. Step 0 is the diagonal tile, which reads
  // only what the wave itself staged, so it runs before the first barrier.
  if (active) phase1(0);
  lds_barrier();
  for (int s = 1; s < nb; ++s) {
    if (active) {
      phase2(s - 1);
      phase1(s);
    }
    lds_barrier();
  }
  if (active) phase2(nb - 1);

  // ---- stores: dQ | dK | dV of the own row, lane dims 16t + 4g .. + 3
  const float cft = __builtin_amdgcn_ldexpf(sum_g(cfa), -kS);
  if (BP && real) {
    // block pairs: each of dQ, dK, dV's HD values of the row (four lanes, DT
    // float4 each) scaled by the power of two that puts their largest |value|
    // at [2^14, 2^15), split to nearest into fp16 hi and lo
    const float f3[3] = {__builtin_amdgcn_ldexpf(sc, -kK - kS), __builtin_amdgcn_ldexpf(sc, -kQ - kS),
                         __builtin_amdgcn_ldexpf(1.f, -kP - kG)};
    const int64_t row = at.row(i);
    unsigned* rowp = reinterpret_cast<unsigned*>(a.qpairs) + row * (3 * int64_t(D) / 8) * 8;
    float* invp = reinterpret_cast<float*>(a.qpairs + a.prows * (3 * int64_t(D) / 8) * 2);
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      const f4* acc = m == 0 ? dq : m == 1 ? dk : dv;
      float v[DT][4];
      float mx = 0.f;
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[t][e] = acc[t][e] * f3[m], mx = fmaxf(mx, fabsf(v[t][e]));
      const float s = pet_split::pair_scale(max_g(mx));
      // lanes g and g ^ 1 (lanes l and l ^ 16) hold the two halves of the
      // 8-value groups 2t + g / 2: the even lane writes the group of each even
      // t, the odd lane that of each odd t, each trading the float4 the other
      // needs, so that every lane stores whole 32-byte groups (hi then lo)
      static_assert(DT % 2 == 0, "groups in lane pairs");
#pragma unroll
      for (int tt = 0; tt < DT; tt += 2) {
        const bool odd = g & 1;
        float x[4], y[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = __shfl_xor(odd ? v[tt][e] : v[tt + 1][e], 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = odd ? x[e] : v[tt][e], y[4 + e] = odd ? v[tt + 1][e] : x[e];
        unsigned h[4], lw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) pet_split::pair2(y[2 * e] * s, y[2 * e + 1] * s, h[e], lw[e]);
        const int col = m * D + at.h * HD + 16 * (tt + (odd ? 1 : 0)) + 8 * (g >> 1);  // the group's first column
        unsigned* hi = rowp + (col >> 3) * 8;
        *reinterpret_cast<u4*>(hi) = u4{h[0], h[1], h[2], h[3]};
        *reinterpret_cast<u4*>(hi + 4) = u4{lw[0], lw[1], lw[2], lw[3]};
      }
      if (g == 0) invp[int64_t(m * H + at.h) * a.prows + row] = 1.f / s;
    }
  } else if (real) {
    float* o = a.qkv_adj + at.row(i) * a.lda + at.h * HD + 4 * g;
    const float fq = __builtin_amdgcn_ldexpf(sc, -kK - kS), fk = __builtin_amdgcn_ldexpf(sc, -kQ - kS);
    const float fv = __builtin_amdgcn_ldexpf(1.f, -kP - kG);
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      *reinterpret_cast<float4*>(o + 16 * t) = make_float4(dq[t][0] * fq, dq[t][1] * fq, dq[t][2] * fq, dq[t][3] * fq);
      *reinterpret_cast<float4*>(o + D + 16 * t) =
          make_float4(dk[t][0] * fk, dk[t][1] * fk, dk[t][2] * fk, dk[t][3] * fk);
      *reinterpret_cast<float4*>(o + 2 * D + 16 * t) =
          make_float4(dv[t][0] * fv, dv[t][1] * fv, dv[t][2] * fv, dv[t][3] * fv);
    }
  }
  if (g == 0 && i < a.S) a.cfh[(size_t(at.n) * H + at.h) * a.S + i] = real ? cft : 0.f;
}

// One workgroup per item. BP: block pairs in place of qkv_adj (a.qpairs).
template <int HD, int NW, bool XF, bool BP = false>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(HD > 32 ? 4 : NW >= 4 ? 6 : 5)))
attn_bwd_pair_kernel(PairBwdArgs a) {
  extern __shared__ float lds_f[];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const Atom at(a.off, xcd_item(blockIdx.x, gridDim.x), a.H, a.N, a.S, a.n0, a.eb);
  PairRows<HD / 4> r;
  pair_bwd_load<HD, XF>(a, at, w, l >> 4, 16 * w + (l & 15), r);
  pair_bwd_item<HD, NW, XF, BP>(a, at, r, reinterpret_cast<unsigned char*>(lds_f));
}

// ---- forward ---------------------------------------------------------------
// The forward at head_dim 32 from the same pairs: a workgroup per (atom,
// head), wave w owning query block w. Per key block J:
//   S^T = K_J Q_w^T on the 16x16x32 instruction (K's rows read straight from
//   the K plane, Q_w split once in registers), a lane holding query 16w + c
//   against keys 16J + 4g + r, so the online softmax reduces across the four
//   g lanes only;
//   O^T += V_J^T P^T on the 16x16x16 instruction, P (scaled by 2^15, split in
//   registers) already its b operand, V^T's a operand transposing reads of the
//   V plane.
// The reference's forward (src/attention.cpp:205-266, :375-449): O_i =
// sum_j softmax_j(sc q_i.k_j + log cf_j) v_j, (max, 1/sum) saved per query.
// LDS: K and V as hi and lo planes, token-major [R slots][HD + 8 halves] (a
// lane's 8 dims one 16-byte store; a key's dims read straight, a dim's four
// keys by the transposing read), log cf of the R slots, each key block's two
// scale exponents: 26.4 KB at five waves and head_dim 32.
struct PairFwdLds {
  int R, PT;
  size_t pl, lc, red, bytes;
  __host__ __device__ constexpr PairFwdLds(int HD, int NW)
      : R(16 * NW), PT(HD + 8), pl(0), lc(size_t(4) * R * PT * 2), red(lc + size_t(R) * 4),
        bytes(red + size_t(8) * NW * 4) {}
};

template <int HD, int NW, bool XF>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(HD <= 32 ? 8 : 5)))
attn_fwd_pair_kernel(const float* __restrict__ qkv, int64_t ldq, const int* __restrict__ off, int N, int n0,
                     int64_t eb, int S, int H, float sc, const float* __restrict__ cf_seq, int64_t ldc,
                     float* __restrict__ merged, int64_t ldm, float* __restrict__ ml, QkvXf xf) {
  // KC 32-dim chunks of the head: lane (c, g) holds dims 32kc + 8g .. + 7 of its row
  constexpr int KC = HD / 32, W = 8 * KC, DT = HD / 16;
  static_assert(HD % 32 == 0, "head_dim a multiple of 32");
  // the fused transform after every row load is issued (one chunk a lane at
  // head_dim 32); at 64 the raw rows held together would spill, so each
  // chunk is transformed as it arrives, branch-free (qkv_get8) so that every
  // chunk's loads are still issued together
  constexpr bool XF_LATE = XF && KC == 1;
  extern __shared__ float lds_f[];
  unsigned char* lds = reinterpret_cast<unsigned char*>(lds_f);
  const int D = H * HD;
  constexpr PairFwdLds L(HD, NW);
  constexpr int PT = L.PT, PS = L.R * PT;  // halves a plane part
  _Float16* KTh = reinterpret_cast<_Float16*>(lds + L.pl);
  _Float16* VTh = KTh + 2 * PS;
  float* lcf = reinterpret_cast<float*>(lds + L.lc);
  float* red = reinterpret_cast<float*>(lds + L.red);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const int i = 16 * w + c;
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, n0, eb);
  const bool active = w < at.nb, real = active && i < at.cnt;

  // own rows (lane (c, g): row 16w + c, dims 32kc + 8g .. + 7); a slot past
  // the count loads slot 0's rows: its key's log cf is kOff (weight exactly 0)
  // and its query's results are not stored
  float q[W], k[W], v[W];
  float pcf = 0.f;
  if (active) {
    const size_t r = at.row(real ? i : 0);
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int col = at.h * HD + 32 * kc + 8 * g;
      if constexpr (XF_LATE) {
        gmem_get<8>(qkv + r * ldq + col, q + 8 * kc);
        gmem_get<8>(qkv + r * ldq + D + col, k + 8 * kc);
        gmem_get<8>(qkv + r * ldq + 2 * D + col, v + 8 * kc);
      } else {
        qkv_get8<XF>(qkv, ldq, r, col, xf, q + 8 * kc);
        qkv_get8<XF>(qkv, ldq, r, D + col, xf, k + 8 * kc);
        qkv_get8<XF>(qkv, ldq, r, 2 * D + col, xf, v + 8 * kc);
      }
    }
    if constexpr (XF_LATE) xf_rows<KC>(xf, r, at.h * HD + 8 * g, D, q, k, v);
    const float c0 = cf_seq[size_t(at.n) * ldc + (real ? i : 0)];
    pcf = real ? c0 : 0.f;
  }
  // Scales per 16-slot block, from the wave's own rows: Q's (this wave's
  // queries), K's and V's (this key block's), each the power of two putting
  // the block's largest row norm at [2^14, 2^15). A block's scores are undone
  // by 2^-(kQ + kK_J); P V accumulates in units of a running V scale 2^kcur,
  // the smallest kV_J seen so far (the largest V), with block J's weights
  // scaled by 2^(15 + kcur - kV_J) <= 2^15 and the accumulator rescaled by a
  // power of two (with the softmax's own rescale) when kcur drops. No
  // workgroup-wide maximum, so a wave computes its own block before the
  // workgroup's only barrier.
  int* kex = reinterpret_cast<int*>(red);  // kK_J at 2J, kV_J at 2J + 1
  float nq = 0.f, nk = 0.f, nv = 0.f;
#pragma unroll
  for (int t = 0; t < W; ++t) nq = fmaf(q[t], q[t], nq), nk = fmaf(k[t], k[t], nk), nv = fmaf(v[t], v[t], nv);
  const int kQ = __builtin_amdgcn_readfirstlane(pair_exp(__builtin_amdgcn_sqrtf(row_max16(sum_g(nq)))));
  const int kKw = __builtin_amdgcn_readfirstlane(pair_exp(__builtin_amdgcn_sqrtf(row_max16(sum_g(nk)))));
  const int kVw = __builtin_amdgcn_readfirstlane(pair_exp(__builtin_amdgcn_sqrtf(row_max16(sum_g(nv)))));
  if (l == 0) kex[2 * w] = kKw, kex[2 * w + 1] = kVw;
  if (g == 0) lcf[i] = pcf > 0.f ? log_cf(pcf) : kOff;
  const float sQ = __builtin_amdgcn_ldexpf(1.f, kQ), sK = __builtin_amdgcn_ldexpf(1.f, kKw);
  const float sV = __builtin_amdgcn_ldexpf(1.f, kVw);
  u4 qb[KC][2];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    u4 kp[2], vp[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int x = 8 * kc + 2 * j;
      unsigned h[3], lo[3];
      pair2s(q[x], q[x + 1], sQ, h[0], lo[0]);
      pair2s(k[x], k[x + 1], sK, h[1], lo[1]);
      pair2s(v[x], v[x + 1], sV, h[2], lo[2]);
      qb[kc][0][j] = h[0], qb[kc][1][j] = lo[0];
      kp[0][j] = h[1], kp[1][j] = lo[1], vp[0][j] = h[2], vp[1][j] = lo[2];
    }
    if (active) {  // the lane's 8 dims of each plane, one 16-byte store
      const int o = tok_off<HD, true>(i, 4 * kc + g);
      *reinterpret_cast<u4*>(KTh + o) = kp[0], *reinterpret_cast<u4*>(KTh + PS + o) = kp[1];
      *reinterpret_cast<u4*>(VTh + o) = vp[0], *reinterpret_cast<u4*>(VTh + PS + o) = vp[1];
    }
  }
  if (!active) {  // slots past the atom's tokens: their sentinel statistics, and the workgroup barrier
    if (ml && g == 0 && i < S) {
      float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
      mlq[0] = kOff, mlq[1] = 0.f;
    }
    lds_barrier();
    return;
  }
  float mx = kFloor, sum = 0.f;
  const float one = opaque_one();
  int kcur = kVw;
  f4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  // block J's scale exponents (the own block's in registers)
  auto kK_of = [&](int J) { return J == w ? kKw : __builtin_amdgcn_readfirstlane(kex[2 * J]); };
  auto kV_of = [&](int J) { return J == w ? kVw : __builtin_amdgcn_readfirstlane(kex[2 * J + 1]); };
  // S^T of key block J: s[r] = query i against key 16J + 4g + r, in 2^(kQ + kK_J) units
  auto scores = [&](int J) {
    f4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      // key 16J + c's dims 32kc + 8g .. + 7, read straight
      const int o = tok_off<HD, true>(16 * J + c, 4 * kc + g);
      const u4 a[2] = {*reinterpret_cast<const u4*>(KTh + o), *reinterpret_cast<const u4*>(KTh + PS + o)};
      st = mfma3(a, qb[kc], st);
    }
    return st;
  };
  // O^T += V_J^T P^T from the block's scaled weights p
  auto pv = [&](int J, const float* p) {
    unsigned h[2], lo[2];
    pair2x(p[0], p[1], one, h[0], lo[0]);
    pair2x(p[2], p[3], one, h[1], lo[1]);
    const u2 ph = {h[0], h[1]}, pl = {lo[0], lo[1]};
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      // dim 16t + c of keys 16J + 4g .. + 3, read transposed (lane 4m + q: key
      // 16J + 4g + m, dims 16t + 4q .. + 3)
      const int o = tok_off<HD, true>(16 * J + 4 * g + (c >> 2), 2 * t + ((c & 3) >> 1)) + 4 * (c & 1);
      acc[t] = mfma3_16(lds_tr16(VTh + o), lds_tr16(VTh + PS + o), ph, pl, acc[t]);
    }
  };
  // the same for two key blocks at once, on the 16x16x32 instruction: k-slots
  // 8g .. 8g + 3 hold block J0's keys 4g .. 4g + 3 and 8g + 4 .. 8g + 7 block
  // J1's, in a and b alike (a contraction is a sum, the slot order is free):
  // three instructions for the two blocks where pv takes six
  auto pv2 = [&](int J0, int J1, const float* p) {
    unsigned h[4], lo[4];
    pair2x(p[0], p[1], one, h[0], lo[0]);
    pair2x(p[2], p[3], one, h[1], lo[1]);
    pair2x(p[4], p[5], one, h[2], lo[2]);
    pair2x(p[6], p[7], one, h[3], lo[3]);
    const u4 ph = {h[0], h[1], h[2], h[3]}, pl = {lo[0], lo[1], lo[2], lo[3]};
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int o0 = tok_off<HD, true>(16 * J0 + 4 * g + (c >> 2), 2 * t + ((c & 3) >> 1)) + 4 * (c & 1);
      const int o1 = tok_off<HD, true>(16 * J1 + 4 * g + (c >> 2), 2 * t + ((c & 3) >> 1)) + 4 * (c & 1);
      const u2 h0 = lds_tr16(VTh + o0), h1 = lds_tr16(VTh + o1);
      const u2 l0 = lds_tr16(VTh + PS + o0), l1 = lds_tr16(VTh + PS + o1);
      const u4 vh = {h0[0], h0[1], h1[0], h1[1]}, vl = {l0[0], l0[1], l1[0], l1[1]};
      acc[t] = pet_split::mfma_h(vl, ph, acc[t]);
      acc[t] = pet_split::mfma_h(vh, pl, acc[t]);
      acc[t] = pet_split::mfma_h(vh, ph, acc[t]);
    }
  };
  auto block = [&](int J, const f4& s) {
    const float scS = __builtin_amdgcn_ldexpf(sc, -kQ - kK_of(J));
    const int kv = kV_of(J);
    const float4 l4 = *reinterpret_cast<const float4*>(lcf + 16 * J + 4 * g);
    const float lc[4] = {l4.x, l4.y, l4.z, l4.w};
    float x[4], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = fmaf(s[r], scS, lc[r]), bm = fmaxf(bm, x[r]);
    const float nm = fmaxf(mx, max_g(bm));
    const float alpha = __expf(mx - nm);
    const int kn = min(kcur, kv);
    float p[4], ps[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __expf(x[r] - nm), ps[r] = __builtin_amdgcn_ldexpf(p[r], 15 + kn - kv);
    sum = fmaf(sum, alpha, (p[0] + p[1]) + (p[2] + p[3]));
    mx = nm;
    const float f = __builtin_amdgcn_ldexpf(alpha, kn - kcur);
    kcur = kn;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= f;
    pv(J, ps);
  };
  auto block2 = [&](int J0, const f4& s0, int J1, const f4& s1) {
    const float sc0 = __builtin_amdgcn_ldexpf(sc, -kQ - kK_of(J0)), sc1 = __builtin_amdgcn_ldexpf(sc, -kQ - kK_of(J1));
    const int kv0 = kV_of(J0), kv1 = kV_of(J1);
    const float4 a4 = *reinterpret_cast<const float4*>(lcf + 16 * J0 + 4 * g);
    const float4 b4 = *reinterpret_cast<const float4*>(lcf + 16 * J1 + 4 * g);
    const float lc[8] = {a4.x, a4.y, a4.z, a4.w, b4.x, b4.y, b4.z, b4.w};
    float x[8], bm = kOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = fmaf(s0[r], sc0, lc[r]), x[4 + r] = fmaf(s1[r], sc1, lc[4 + r]);
      bm = fmaxf(bm, fmaxf(x[r], x[4 + r]));
    }
    const float nm = fmaxf(mx, max_g(bm));
    const float alpha = __expf(mx - nm);
    const int kn = min(kcur, min(kv0, kv1));
    float p[8], ps[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = __expf(x[r] - nm), ps[r] = __builtin_amdgcn_ldexpf(p[r], 15 + kn - kv0);
      p[4 + r] = __expf(x[4 + r] - nm), ps[4 + r] = __builtin_amdgcn_ldexpf(p[4 + r], 15 + kn - kv1);
    }
    sum = fmaf(sum, alpha, ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
    mx = nm;
    const float f = __builtin_amdgcn_ldexpf(alpha, kn - kcur);
    kcur = kn;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= f;
    pv2(J0, J1, ps);
  };
  // the own key block first (the wave staged it itself), before the barrier;
  // then the others w + 1, w + 2, ... (mod nb), two at a time, an odd one last
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
  // a query on an edge at its cutoff gets zeros
  const bool live = real && (i == 0 || !is_off(lcf[i]));
  const float invl = live && tot > 0.f ? 1.0f / tot : 0.f;
  const float mxs = live && tot > 0.f ? mx : kOff;  // no live key: the max never left kFloor
  if (real) {
    const float f = __builtin_amdgcn_ldexpf(invl, -15 - kcur);
    float* o = merged + at.grow(i) * ldm + at.h * HD + 4 * g;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4*>(o + 16 * t) = make_float4(acc[t][0] * f, acc[t][1] * f, acc[t][2] * f, acc[t][3] * f);
  }
  if (ml && g == 0 && i < S) {
    float* mlq = ml + 2 * ((size_t(at.n) * H + at.h) * S + i);
    mlq[0] = real ? mxs : kOff, mlq[1] = real ? invl : 0.f;
  }
}

// ---- host side ---------------------------------------------------------------

size_t pair_bwd_bytes(int HD, int NW) { return NW <= kPairMaxWaves ? PairLds(HD, NW).bytes : ~size_t(0); }

const void* pair_bwd_kernel_ptr(int HD) {
  return HD == 64 ? reinterpret_cast<const void*>(attn_bwd_pair_kernel<64, 5, false>)
                  : reinterpret_cast<const void*>(attn_bwd_pair_kernel<32, 5, false>);
}

namespace {
template <int HD, int NW, bool BP = false>
const void* pair_kernel(bool x) {
  return x ? reinterpret_cast<const void*>(attn_bwd_pair_kernel<HD, NW, true, BP>)
           : reinterpret_cast<const void*>(attn_bwd_pair_kernel<HD, NW, false, BP>);
}
template <int HD, bool BP = false>
const void* pair_kernel_nw(int NW, bool x) {
  switch (NW) {
    case 1: return pair_kernel<HD, 1, BP>(x);
    case 2: return pair_kernel<HD, 2, BP>(x);
    case 3: return pair_kernel<HD, 3, BP>(x);
    case 4: return pair_kernel<HD, 4, BP>(x);
    case 5: return pair_kernel<HD, 5, BP>(x);
    case 6: return pair_kernel<HD, 6, BP>(x);
    case 7: return pair_kernel<HD, 7, BP>(x);
    default: return pair_kernel<HD, 8, BP>(x);
  }
}

// The dynamic LDS limit of kernel k raised, once per device, to the largest
// size asked.
int allow_lds_pair(const void* k, size_t bytes) {
  if (bytes <= 65536) return PET_ATTN_OK;
  static std::map<std::pair<int, const void*>, size_t> raised;
  static std::mutex mu;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return PET_ATTN_ELAUNCH;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = raised[{dev, k}];
  if (have < bytes) {
    if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)) != hipSuccess)
      return PET_ATTN_ELAUNCH;
    have = bytes;
  }
  return PET_ATTN_OK;
}
}  // namespace

int pair_bwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
             const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
             const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh, QkvXf xf, hipStream_t st,
             void* qpairs, int64_t prows) {
  const int NW = (sh.slots + 15) / 16, HD = sh.head_dim;
  if (NW > kPairMaxWaves || (HD != 32 && HD != 64)) return PET_ATTN_ESLOTS;
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  if (items > INT32_MAX) return PET_ATTN_EINVAL;
  const size_t bytes = pair_bwd_bytes(HD, NW);
  const bool x = xf.rs || xf.b;
  const void* k = qpairs ? (HD == 64 ? pair_kernel_nw<64, true>(NW, x) : pair_kernel_nw<32, true>(NW, x))
                         : (HD == 64 ? pair_kernel_nw<64>(NW, x) : pair_kernel_nw<32>(NW, x));
  if (const int e = allow_lds_pair(k, bytes)) return e;
  const PairBwdArgs a{qkv,  ldq,    off,    sh.n_atoms, n0,  eb,   sh.slots, sh.heads,
                      sh.scale, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, xf,
                      static_cast<u4*>(qpairs), prows};
  void* args[] = {const_cast<PairBwdArgs*>(&a)};
  if (hipLaunchKernel(k, dim3(unsigned(items)), dim3(64 * NW), args, bytes, st) != hipSuccess) return PET_ATTN_ELAUNCH;
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

size_t pair_fwd_bytes(int HD, int NW) { return NW <= kPairMaxWaves ? PairFwdLds(HD, NW).bytes : ~size_t(0); }

const void* pair_fwd_kernel_ptr(int HD) {
  return HD == 64 ? reinterpret_cast<const void*>(attn_fwd_pair_kernel<64, 5, false>)
                  : reinterpret_cast<const void*>(attn_fwd_pair_kernel<32, 5, false>);
}

int pair_fwd(const pet_attn_shape& sh, int n0, int n1, int64_t eb, const float* qkv, int64_t ldq, const int* off,
             const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, QkvXf xf, hipStream_t st) {
  const int NW = (sh.slots + 15) / 16, HD = sh.head_dim;
  if (NW > kPairMaxWaves || (HD != 32 && HD != 64)) return PET_ATTN_ESLOTS;
  const int64_t items = int64_t(n1 - n0) * sh.heads;
  if (items == 0) return PET_ATTN_OK;
  const bool x = xf.rs || xf.b;
  const size_t bytes = pair_fwd_bytes(HD, NW);
  decltype(&attn_fwd_pair_kernel<32, 1, false>) k = nullptr;
  auto pick = [&](auto hd, auto nw) {
    constexpr int D_ = decltype(hd)::value, V = decltype(nw)::value;
    k = x ? attn_fwd_pair_kernel<D_, V, true> : attn_fwd_pair_kernel<D_, V, false>;
  };
  auto by_waves = [&](auto hd) {
    switch (NW) {
      case 1: pick(hd, std::integral_constant<int, 1>{}); break;
      case 2: pick(hd, std::integral_constant<int, 2>{}); break;
      case 3: pick(hd, std::integral_constant<int, 3>{}); break;
      case 4: pick(hd, std::integral_constant<int, 4>{}); break;
      case 5: pick(hd, std::integral_constant<int, 5>{}); break;
      case 6: pick(hd, std::integral_constant<int, 6>{}); break;
      case 7: pick(hd, std::integral_constant<int, 7>{}); break;
      default: pick(hd, std::integral_constant<int, 8>{}); break;
    }
  };
  if (HD == 64)
    by_waves(std::integral_constant<int, 64>{});
  else
    by_waves(std::integral_constant<int, 32>{});
  if (const int e = allow_lds_pair(reinterpret_cast<const void*>(k), bytes)) return e;
  hipLaunchKernelGGL(k, dim3(unsigned(items)), dim3(64 * NW), bytes, st, qkv, ldq, off, sh.n_atoms, n0, eb, sh.slots,
                     sh.heads, sh.scale, cf_seq, ldc, merged, ldm, ml, xf);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

}  // namespace pet_attn
