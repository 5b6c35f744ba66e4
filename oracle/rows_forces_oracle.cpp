// TEST INFRASTRUCTURE ONLY -- the CPU oracle of the attention's input side
// (cf_seq, the token norm) and of the consumer of its cf adjoint (the forces'
// edge term, the fold, the sum over structures).
//
// A restatement, in this repository's own code, of the reference's host paths
// of peterspackman/pet-kokkos; the checker the HIP kernels are compared with.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
//
// What each function follows (file:line in the reference tree):
//   cf_seq          pet_cfseq / cf build          src/device_neighbors.cpp:318-323,
//                                                 src/model.cpp:375-377
//   norm_rows       norm_rows (Kokkos passes)     src/ops.hpp:376-407; eps :195-196
//   norm_rows_bwd   norm_rows_bwd                 src/ops.hpp:409-436, grad() :294-298
//   cutoff value    dev_{bump,cosine,smooth}_cutoff  include/pet/cutoff.hpp:17-35
//   cutoff_ddist    bump/cosine/smooth_ddist      src/forces.cpp:21-42
//   edge_grad       forces_and_virial "edge_grad" src/forces.cpp:364-378
//   fold            fold_edge_gradients           src/forces.cpp:50-68
//   struct_sum      sum_by_structure              src/forces.cpp:287-302
// The norm has an fp64 twin for the library and finite-difference checks; the
// cutoff functions an fp64 variant (all arithmetic in double) for the
// finite-difference checks of their derivatives. The pins of each function are
// in tests/test_oracle_rows_forces.py.
#include <cmath>
#include <cstdint>

namespace {

constexpr double kPi = 3.14159265358979323846;

template <class R>
void norm_rows(int rows, int D, R* out, int64_t ldo, const R* in, int64_t ldi, const R* w, const R* b) {
  const bool ln = b != nullptr;
  const R eps = ln ? R(1e-5) : R(1.1920928955078125e-07);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const R* x = in + int64_t(r) * ldi;
    R mu = R(0);
    if (ln) {
      R s = R(0);
      for (int d = 0; d < D; ++d) s += x[d];
      mu = s / R(D);
    }
    R v = R(0);
    for (int d = 0; d < D; ++d) v += (x[d] - mu) * (x[d] - mu);
    const R inv = R(1) / std::sqrt(v / R(D) + eps);
    for (int d = 0; d < D; ++d) out[int64_t(r) * ldo + d] = (x[d] - mu) * inv * w[d] + (ln ? b[d] : R(0));
  }
}

template <class R>
void norm_rows_bwd(int rows, int D, R* in_adj, int64_t lda, R beta, const R* g, int64_t ldg, const R* in,
                   int64_t ldi, const R* w, bool ln) {
  const R eps = ln ? R(1e-5) : R(1.1920928955078125e-07);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const R* x = in + int64_t(r) * ldi;
    const R* ga = g + int64_t(r) * ldg;
    R mu = R(0);
    if (ln) {
      R s = R(0);
      for (int d = 0; d < D; ++d) s += x[d];
      mu = s / R(D);
    }
    R sq = R(0), sg = R(0), sgx = R(0);
    for (int d = 0; d < D; ++d) {
      const R xv = x[d] - mu, gw = ga[d] * w[d];
      sq += xv * xv;
      sg += gw;
      sgx += gw * xv;
    }
    const R inv = R(1) / std::sqrt(sq / R(D) + eps);
    const R mg = ln ? sg / R(D) : R(0), mgx = sgx * inv / R(D);
    R* a = in_adj + int64_t(r) * lda;
    for (int d = 0; d < D; ++d) {
      const R gd = inv * (ga[d] * w[d] - mg - (x[d] - mu) * inv * mgx);
      a[d] = beta == R(0) ? gd : beta * a[d] + gd;
    }
  }
}

// The cutoff factors and their distance derivatives; T is the type of the
// transcendentals (float as the reference's CutT, or double for the
// finite-difference checks).
template <class T>
double cutoff_value(double d, double rc, double w, int kind) {
  if (kind == 0) {
    const T x = T((d - (rc - w)) / w);
    if (x <= T(0)) return 1.0;
    if (x >= T(1)) return 0.0;
    return 0.5 * (1.0 + double(std::tanh(T(1) / std::tan(T(kPi) * x))));
  }
  if (kind == 1) {
    const T x = std::fmin(std::fmax(T((d - (rc - w)) / w), T(0)), T(1));
    return 0.5 * (1.0 + double(std::cos(T(kPi) * x)));
  }
  const double x = std::fmin(std::fmax((d - (rc - w)) / w, 0.0), 1.0);
  const double x4 = x * x * x * x;
  return 1.0 - x4 * (35.0 - 84.0 * x + 70.0 * x * x - 20.0 * x * x * x);
}

template <class T>
double cutoff_ddist(double d, double rc, double w, int kind) {
  if (kind == 0) {
    const T x = T((d - (rc - w)) / w);
    if (x <= T(0) || x >= T(1)) return 0.0;
    const T si = std::sin(T(kPi) * x);
    const T t = std::tanh(std::cos(T(kPi) * x) / si);
    const T du = (-T(kPi) / (si * si)) / T(w);
    return 0.5 * (1.0 - double(t * t)) * double(du);
  }
  if (kind == 1) {
    const T x = T((d - (rc - w)) / w);
    if (x <= T(0) || x >= T(1)) return 0.0;
    return 0.5 * double(-T(kPi) * std::sin(T(kPi) * x)) / w;
  }
  const double x = (d - (rc - w)) / w;
  if (x <= 0.0 || x >= 1.0) return 0.0;
  const double y = x * (1.0 - x);
  return -140.0 * y * y * y / w;
}

}  // namespace

extern "C" {

#define ORACLE_EXPORT __attribute__((visibility("default")))

ORACLE_EXPORT void oracle_cf_seq(int N, int S, const int* off, const float* cut, float* cf_seq, int64_t ldc) {
  for (int n = 0; n < N; ++n)
    for (int s = 0; s < S; ++s) {
      const int cnt = off[n + 1] - off[n] + 1;
      cf_seq[int64_t(n) * ldc + s] = s == 0 ? 1.0f : s < cnt ? cut[off[n] + s - 1] : 0.0f;
    }
}

ORACLE_EXPORT void oracle_norm_rows_f32(int rows, int D, float* out, int64_t ldo, const float* in, int64_t ldi,
                                        const float* w, const float* b) {
  norm_rows<float>(rows, D, out, ldo, in, ldi, w, b);
}
ORACLE_EXPORT void oracle_norm_rows_f64(int rows, int D, double* out, int64_t ldo, const double* in, int64_t ldi,
                                        const double* w, const double* b) {
  norm_rows<double>(rows, D, out, ldo, in, ldi, w, b);
}
ORACLE_EXPORT void oracle_norm_rows_bwd_f32(int rows, int D, float* in_adj, int64_t lda, float beta, const float* g,
                                            int64_t ldg, const float* in, int64_t ldi, const float* w, int ln) {
  norm_rows_bwd<float>(rows, D, in_adj, lda, beta, g, ldg, in, ldi, w, ln != 0);
}
ORACLE_EXPORT void oracle_norm_rows_bwd_f64(int rows, int D, double* in_adj, int64_t lda, double beta,
                                            const double* g, int64_t ldg, const double* in, int64_t ldi,
                                            const double* w, int ln) {
  norm_rows_bwd<double>(rows, D, in_adj, lda, beta, g, ldg, in, ldi, w, ln != 0);
}

// cutoff values / derivatives at n distances; f64 nonzero: transcendentals in double
ORACLE_EXPORT void oracle_cutoff(int n, const double* d, const double* rc, double w, int kind, int f64,
                                 double* value, double* ddist) {
  for (int i = 0; i < n; ++i) {
    if (value) value[i] = f64 ? cutoff_value<double>(d[i], rc[i], w, kind) : cutoff_value<float>(d[i], rc[i], w, kind);
    if (ddist) ddist[i] = f64 ? cutoff_ddist<double>(d[i], rc[i], w, kind) : cutoff_ddist<float>(d[i], rc[i], w, kind);
  }
}

ORACLE_EXPORT void oracle_edge_grad(int nc, int E, const int* off, const int* center, const float* x4_adj,
                                    int64_t ldx, const float* cutoff_adj, const float* cf_seq_adj, int64_t ldca,
                                    const double* vec, const double* dist, const double* pcut, double width, int kind,
                                    double* grad) {
  for (int k = 0; k < E; ++k) {
    if (k >= off[nc]) {
      grad[3 * k] = grad[3 * k + 1] = grad[3 * k + 2] = 0.0;
      continue;
    }
    const int n = center[k], m = k - off[n];
    const float* xa = x4_adj + int64_t(k) * ldx;
    const double cutoff_total = (cutoff_adj ? cutoff_adj[k] : 0.0f) + cf_seq_adj[int64_t(n) * ldca + 1 + m];
    const double dcut_dd = cutoff_ddist<float>(dist[k], pcut[k], width, kind);
    const double dist_adj = xa[3] + cutoff_total * dcut_dd;
    const double invd = dist[k] > 0.0 ? 1.0 / dist[k] : 0.0;
    for (int c = 0; c < 3; ++c) grad[3 * k + c] = xa[c] + dist_adj * vec[3 * k + c] * invd;
  }
}

ORACLE_EXPORT void oracle_fold(int N, int nc, const int* off, const int* rev, const double* vec, const double* grad,
                               double scale, double* forces, double* vir) {
  for (int i = 0; i < N; ++i) {
    double f[3] = {0, 0, 0}, w[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = i < nc ? off[i] : 0; k < (i < nc ? off[i + 1] : 0); ++k) {
      for (int c = 0; c < 3; ++c) f[c] += grad[3 * k + c];
      for (int a = 0; a < 3; ++a)
        for (int b = 0; b < 3; ++b) w[a * 3 + b] += vec[3 * k + a] * grad[3 * k + b];
      if (rev[k] >= 0)
        for (int c = 0; c < 3; ++c) f[c] -= grad[3 * rev[k] + c];
    }
    for (int c = 0; c < 3; ++c) forces[3 * i + c] = scale * f[c];
    for (int t = 0; t < 9; ++t) vir[9 * i + t] = scale * w[t];
  }
}

ORACLE_EXPORT void oracle_struct_sum(int NS, int width, const int* soff, const double* x, double* out, int acc) {
  for (int b = 0; b < NS; ++b)
    for (int t = 0; t < width; ++t) {
      double s = 0.0;
      for (int a = soff[b]; a < soff[b + 1]; ++a) s += x[int64_t(a) * width + t];
      out[b * width + t] = acc ? out[b * width + t] + s : s;
    }
}

}  // extern "C"
