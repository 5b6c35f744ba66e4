// TEST INFRASTRUCTURE ONLY -- the CPU oracle of PET's neighbourhood attention.
//
// A restatement, in this repository's own code, of the reference's host
// (OpenMP "flat") attention path of peterspackman/pet-kokkos: one work item
// per (atom, head, slot), the keys read straight from the token matrix. It is
// the checker the HIP kernels are compared with; only tests/, the smoke check
// of __graft_entry__.py and bench.py's cpu_baseline leg load it. The product
// library never links it and has no CPU fallback.
//
// What each function follows (file:line in the reference tree):
//   fwd_token      Forward<HD>::token            src/attention.cpp:217-248
//   queries_token  Queries<HD>::token            src/attention.cpp:1579-1601
//   keys_token     Keys<HD, true, true>::token   src/attention.cpp:1637-1673
//                  (the host runs one keys pass, split = false, :1892-1904)
//   cf_adjoint     the attn_bwd_cf lambda        src/attention.cpp:1829-1838
//   zero_dead      zero_dead                     src/attention.cpp:1510-1518
//   linear         out = in W^T + b (+beta out)  src/ops.hpp:41-44, src/ops.cpp:24
//   linear_bwd     in_adj = out_adj W (+beta)    src/ops.hpp:44-45, src/ops.cpp:50-52
//   Tokens         count(n), row(n, s)           src/ops.hpp:31-37
//   constants      kOff = -1e30, off: < -1e29    src/attention.cpp:54-55
//   exp / log      host fast_exp/fast_log = expf/logf (exp/log in fp64)
//                                                include/pet/kokkos.hpp:263-278
//   dot_row        four products per step when head_dim % 4 == 0
//                                                src/attention.cpp:124-135
// Every function has an fp64 twin (the _f64 exports) for the brute-force and
// finite-difference checks. The pins of each function are listed in
// tests/test_oracle.py; none of them is "parity unpinned".
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../include/pet_attn.h"

namespace {

template <class R>
inline R xexp(R x);
template <>
inline float xexp<float>(float x) { return expf(x); }
template <>
inline double xexp<double>(double x) { return std::exp(x); }
template <class R>
inline R xlog(R x);
template <>
inline float xlog<float>(float x) { return logf(x); }
template <>
inline double xlog<double>(double x) { return std::log(x); }

template <class R>
constexpr R kOff = R(-1e30);
template <class R>
inline bool is_off(R lc) { return lc < R(-1e29); }

struct Tok {
  const int* off;
  int N;
  int count(int n) const { return off[n + 1] - off[n] + 1; }
  int64_t row(int n, int s) const { return s == 0 ? n : int64_t(N) + off[n] + s - 1; }
};

// row . reg over a head's slice, four products a step where hd allows.
template <class R>
inline R dot_row(const R* row, const R* reg, int nd) {
  R s = R(0);
  if (nd % 4 == 0) {
    for (int d = 0; d < nd; d += 4) s += row[d] * reg[d] + row[d + 1] * reg[d + 1] + row[d + 2] * reg[d + 2] + row[d + 3] * reg[d + 3];
  } else {
    for (int d = 0; d < nd; ++d) s += row[d] * reg[d];
  }
  return s;
}
template <class R>
inline void axpby_row(R* acc, R c, R p, const R* row, int nd) {
  for (int d = 0; d < nd; ++d) acc[d] = acc[d] * c + p * row[d];
}
template <class R>
inline R log_cf(R cf) { return cf > R(0) ? xlog<R>(cf) : kOff<R>; }

constexpr int kMaxHd = 128;

// ---- forward ---------------------------------------------------------------
template <class R>
void fwd(const pet_attn_shape& sh, const R* qkv, int64_t ldq, const int* off, const R* cf_seq, int64_t ldc,
         R* merged, int64_t ldm, R* ml) {
  const int N = sh.n_atoms, H = sh.heads, S = sh.slots, hd = sh.head_dim, D = H * hd;
  const R sc = R(sh.scale);
  const Tok tk{off, N};
  const int64_t total = int64_t(N) * H * S;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; ++i) {
    const int sq = int(i % S), h = int((i / S) % H), n = int(i / (int64_t(S) * H));
    const int qo = h * hd, cnt = tk.count(n);
    const R* cf = cf_seq + int64_t(n) * ldc;
    R* mlq = ml ? ml + 2 * i : nullptr;
    if (sq >= cnt) {  // a slot past the atom's tokens
      if (mlq) mlq[0] = kOff<R>, mlq[1] = R(0);
      continue;
    }
    const int64_t rq = tk.row(n, sq);
    if (sq > 0 && is_off(log_cf(cf[sq]))) {  // a query on an edge at its cutoff
      for (int d = 0; d < hd; ++d) merged[rq * ldm + qo + d] = R(0);
      if (mlq) mlq[0] = kOff<R>, mlq[1] = R(0);
      continue;
    }
    R q[kMaxHd], acc[kMaxHd];
    for (int d = 0; d < hd; ++d) q[d] = qkv[rq * ldq + qo + d], acc[d] = R(0);
    R mx = kOff<R>, l = R(0);
    for (int k = 0; k < cnt; ++k) {
      const R lc = log_cf(cf[k]);
      if (is_off(lc)) continue;
      const int64_t rk = tk.row(n, k);
      const R s = dot_row(qkv + rk * ldq + D + qo, q, hd) * sc + lc;
      const R nm = s > mx ? s : mx;
      const R c = xexp<R>(mx - nm), p = xexp<R>(s - nm);
      l = l * c + p;
      axpby_row(acc, c, p, qkv + rk * ldq + 2 * D + qo, hd);
      mx = nm;
    }
    const R invl = l > R(0) ? R(1) / l : R(0);
    for (int d = 0; d < hd; ++d) merged[rq * ldm + qo + d] = acc[d] * invl;
    if (mlq) mlq[0] = mx, mlq[1] = invl;
  }
}

template <class R>
void zero_dead(R* x, int64_t ld, int width, int N, int T, const int* off, int dead) {
  if (!dead) return;
  for (int64_t r = int64_t(N) + off[N]; r < T; ++r)
    for (int c = 0; c < width; ++c) x[r * ld + c] = R(0);
}

// ---- backward --------------------------------------------------------------
template <class R>
void bwd(const pet_attn_shape& sh, const R* qkv, int64_t ldq, const int* off, const R* dmerged, int64_t ldg,
         const R* merged, int64_t ldm, const R* ml, const R* cf_seq, int64_t ldc, R* qkv_adj, int64_t lda, R* cfh,
         R* cf_seq_adj, int64_t ldca) {
  const int N = sh.n_atoms, H = sh.heads, S = sh.slots, hd = sh.head_dim, D = H * hd;
  const R sc = R(sh.scale);
  const Tok tk{off, N};
  const int64_t total = int64_t(N) * H * S;
  R* dq_out = new R[total > 0 ? total : 1];
  // Queries: Dq = dO . O, dQ = sc sum_k A (dO . v_k - Dq) k_k.
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; ++i) {
    const int sq = int(i % S), h = int((i / S) % H), n = int(i / (int64_t(S) * H));
    const int qo = h * hd, cnt = tk.count(n);
    if (sq >= cnt) {
      dq_out[i] = R(0);
      continue;
    }
    const R* cf = cf_seq + int64_t(n) * ldc;
    const int64_t rq = tk.row(n, sq);
    const R m = ml[2 * i], invl = ml[2 * i + 1];
    R q[kMaxHd], dout[kMaxHd], dq[kMaxHd];
    for (int d = 0; d < hd; ++d) q[d] = qkv[rq * ldq + qo + d], dout[d] = dmerged[rq * ldg + qo + d], dq[d] = R(0);
    const R Dq = dot_row(merged + rq * ldm + qo, dout, hd);
    dq_out[i] = Dq;
    if (invl > R(0))
      for (int k = 0; k < cnt; ++k) {
        const R lc = log_cf(cf[k]);
        if (is_off(lc)) continue;
        const int64_t rk = tk.row(n, k);
        const R* K = qkv + rk * ldq + D + qo;
        const R a = xexp<R>(dot_row(K, q, hd) * sc + lc - m) * invl;
        const R ds = a * (dot_row(qkv + rk * ldq + 2 * D + qo, dout, hd) - Dq) * sc;
        axpby_row(dq, R(1), ds, K, hd);
      }
    for (int d = 0; d < hd; ++d) qkv_adj[rq * lda + qo + d] = dq[d];
  }
  // Keys: dK = sc sum_q dS q_q, dV = sum_q A dO_q, and the key's dS summed.
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < total; ++i) {
    const int sk = int(i % S), h = int((i / S) % H), n = int(i / (int64_t(S) * H));
    const int cnt = tk.count(n), ko = D + h * hd, vo = 2 * D + h * hd;
    const int64_t b = (int64_t(n) * H + h) * S;
    if (sk >= cnt) {
      cfh[(int64_t(n) * S + sk) * H + h] = R(0);
      continue;
    }
    const int64_t rk = tk.row(n, sk);
    R k[kMaxHd], v[kMaxHd], dk[kMaxHd], dv[kMaxHd];
    for (int d = 0; d < hd; ++d) dk[d] = R(0), dv[d] = R(0);
    R cf_acc = R(0);
    const R cf = cf_seq[int64_t(n) * ldc + sk];
    if (cf > R(0)) {
      const R lcf = xlog<R>(cf);
      for (int d = 0; d < hd; ++d) k[d] = qkv[rk * ldq + ko + d], v[d] = qkv[rk * ldq + vo + d];
      for (int q = 0; q < cnt; ++q) {
        const R invl = ml[2 * (b + q) + 1];
        if (invl <= R(0)) continue;
        const int64_t rq = tk.row(n, q);
        const R* Q = qkv + rq * ldq + h * hd;
        const R* G = dmerged + rq * ldg + h * hd;
        const R a = xexp<R>(dot_row(Q, k, hd) * sc + lcf - ml[2 * (b + q)]) * invl;
        const R ds = a * (dot_row(G, v, hd) - dq_out[b + q]);
        axpby_row(dk, R(1), ds * sc, Q, hd);
        axpby_row(dv, R(1), a, G, hd);
        cf_acc += ds;
      }
    }
    for (int d = 0; d < hd; ++d) qkv_adj[rk * lda + ko + d] = dk[d], qkv_adj[rk * lda + vo + d] = dv[d];
    cfh[(int64_t(n) * S + sk) * H + h] = cf_acc;
  }
  delete[] dq_out;
  // The cf adjoint: heads summed in order, divided by cf, accumulated.
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < int64_t(N) * S; ++i) {
    const int sk = int(i % S), n = int(i / S);
    const R cf = cf_seq[int64_t(n) * ldc + sk];
    if (cf <= R(0)) continue;
    R total_h = R(0);
    for (int h = 0; h < H; ++h) total_h += cfh[(int64_t(n) * S + sk) * H + h];
    cf_seq_adj[int64_t(n) * ldca + sk] += total_h / cf;
  }
  zero_dead(qkv_adj, lda, 3 * D, N, sh.n_rows, off, sh.dead);
}

// out[M, Nout] = in[M, K] W[Nout, K]^T + b, onto beta out; fp64 accumulation.
template <class R>
void linear(R* out, int64_t ldo, const R* in, int64_t ldi, const R* W, const R* b, int M, int Nout, int K, R beta) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i)
    for (int j = 0; j < Nout; ++j) {
      double s = b ? double(b[j]) : 0.0;
      const R* x = in + i * ldi;
      const R* w = W + int64_t(j) * K;
      for (int k = 0; k < K; ++k) s += double(x[k]) * double(w[k]);
      R* o = out + i * ldo + j;
      *o = R(s) + (beta != R(0) ? beta * *o : R(0));
    }
}
// in_adj[M, K] = out_adj[M, Nout] W[Nout, K], onto beta in_adj; fp64 accumulation.
template <class R>
void linear_bwd(R* in_adj, int64_t ldi, const R* out_adj, int64_t ldo, const R* W, int M, int Nout, int K, R beta) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M; ++i) {
    double acc[1024];
    for (int kb = 0; kb < K; kb += 1024) {
      const int kw = K - kb < 1024 ? K - kb : 1024;
      for (int k = 0; k < kw; ++k) acc[k] = 0.0;
      for (int j = 0; j < Nout; ++j) {
        const double g = double(out_adj[i * ldo + j]);
        const R* w = W + int64_t(j) * K + kb;
        for (int k = 0; k < kw; ++k) acc[k] += g * double(w[k]);
      }
      for (int k = 0; k < kw; ++k) {
        R* o = in_adj + i * ldi + kb + k;
        *o = R(acc[k]) + (beta != R(0) ? beta * *o : R(0));
      }
    }
  }
}

}  // namespace

extern "C" {

#define ORACLE_EXPORT __attribute__((visibility("default")))

ORACLE_EXPORT int oracle_attn_fwd_f32(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off,
                                      const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml) {
  fwd<float>(*sh, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml);
  zero_dead(merged, ldm, sh->heads * sh->head_dim, sh->n_atoms, sh->n_rows, off, sh->dead);
  return 0;
}
ORACLE_EXPORT int oracle_attn_fwd_f64(const pet_attn_shape* sh, const double* qkv, int64_t ldq, const int* off,
                                      const double* cf_seq, int64_t ldc, double* merged, int64_t ldm, double* ml) {
  fwd<double>(*sh, qkv, ldq, off, cf_seq, ldc, merged, ldm, ml);
  zero_dead(merged, ldm, sh->heads * sh->head_dim, sh->n_atoms, sh->n_rows, off, sh->dead);
  return 0;
}
ORACLE_EXPORT int oracle_attn_bwd_f32(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const int* off,
                                      const float* dmerged, int64_t ldg, const float* merged, int64_t ldm,
                                      const float* ml, const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda,
                                      float* cfh, float* cf_seq_adj, int64_t ldca) {
  bwd<float>(*sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, cf_seq_adj, ldca);
  return 0;
}
ORACLE_EXPORT int oracle_attn_bwd_f64(const pet_attn_shape* sh, const double* qkv, int64_t ldq, const int* off,
                                      const double* dmerged, int64_t ldg, const double* merged, int64_t ldm,
                                      const double* ml, const double* cf_seq, int64_t ldc, double* qkv_adj,
                                      int64_t lda, double* cfh, double* cf_seq_adj, int64_t ldca) {
  bwd<double>(*sh, qkv, ldq, off, dmerged, ldg, merged, ldm, ml, cf_seq, ldc, qkv_adj, lda, cfh, cf_seq_adj, ldca);
  return 0;
}
ORACLE_EXPORT void oracle_linear_f32(float* out, int64_t ldo, const float* in, int64_t ldi, const float* W,
                                     const float* b, int M, int Nout, int K, float beta) {
  linear<float>(out, ldo, in, ldi, W, b, M, Nout, K, beta);
}
ORACLE_EXPORT void oracle_linear_bwd_f32(float* in_adj, int64_t ldi, const float* out_adj, int64_t ldo,
                                         const float* W, int M, int Nout, int K, float beta) {
  linear_bwd<float>(in_adj, ldi, out_adj, ldo, W, M, Nout, K, beta);
}

// attention(): the forward, zero_dead, then out = merged W_out^T + b_out.
// (reference src/attention.cpp:1520-1558, finish() at :1529-1532)
ORACLE_EXPORT int oracle_attention_f32(const pet_attn_shape* sh, float* out, int64_t ldo, const float* qkv,
                                       int64_t ldq, const float* cf_seq, int64_t ldc, const float* w_out,
                                       const float* b_out, const int* off, float* merged, float* ml) {
  const int D = sh->heads * sh->head_dim;
  oracle_attn_fwd_f32(sh, qkv, ldq, off, cf_seq, ldc, merged, D, ml);
  linear<float>(out, ldo, merged, D, w_out, b_out, sh->n_rows, D, D, 0.0f);
  return 0;
}
// attention_bwd(): dmerged = out_adj W_out, the core backward, the cf adjoint,
// zero_dead, in_adj = qkv_adj W_in + beta in_adj.
// (reference src/attention.cpp:1814-1907)
ORACLE_EXPORT int oracle_attention_bwd_f32(const pet_attn_shape* sh, float* in_adj, int64_t ldi, int d_in,
                                           float* cf_seq_adj, int64_t ldca, const float* out_adj, int64_t ldo,
                                           const float* qkv, int64_t ldq, const float* cf_seq, int64_t ldc,
                                           const float* w_in, const float* w_out, const int* off,
                                           const float* merged, const float* ml, float beta) {
  const int D = sh->heads * sh->head_dim, T = sh->n_rows, N = sh->n_atoms, S = sh->slots, H = sh->heads;
  float* dmerged = new float[int64_t(T) * D];
  float* qkv_adj = new float[int64_t(T) * 3 * D];
  float* cfh = new float[int64_t(N) * S * H + 1];
  linear_bwd<float>(dmerged, D, out_adj, ldo, w_out, T, D, D, 0.0f);
  bwd<float>(*sh, qkv, ldq, off, dmerged, D, merged, D, ml, cf_seq, ldc, qkv_adj, 3 * D, cfh, cf_seq_adj, ldca);
  linear_bwd<float>(in_adj, ldi, qkv_adj, 3 * D, w_in, T, 3 * D, d_in, beta);
  delete[] dmerged;
  delete[] qkv_adj;
  delete[] cfh;
  return 0;
}

}  // extern "C"
