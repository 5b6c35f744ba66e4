// The consumer of the attention's cf adjoint on gfx950: the per-edge gradient
// of forces_and_virial (peterspackman/pet-kokkos src/forces.cpp:364-378), the
// fold of edge gradients into forces and per-atom virials (:50-68) and the sum
// over structures (:287-302).
//
// These passes are small and memory-bound (a few hundred bytes an edge at
// most); their contract is the arithmetic: fp64 sums with the cutoff's
// derivative in fp32 as the reference's CutT evaluates it, and fixed summation
// orders so the bits repeat from run to run.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/pet_attn.h"

namespace pet_forces {

constexpr double kPi = 3.14159265358979323846;

// d cf / d dist of the three smooth cutoffs (src/forces.cpp:21-40): the
// transcendentals in float, the rest in double, in the reference's order.
__device__ __forceinline__ double bump_ddist(double d, double rc, double w) {
  const float x = float((d - (rc - w)) / w);
  if (x <= 0.0f || x >= 1.0f) return 0.0;
  const float si = sinf(float(kPi) * x);
  const float t = tanhf(cosf(float(kPi) * x) / si);
  const float du = (-float(kPi) / (si * si)) / float(w);
  return 0.5 * (1.0 - double(t * t)) * double(du);
}
__device__ __forceinline__ double cosine_ddist(double d, double rc, double w) {
  const float x = float((d - (rc - w)) / w);
  if (x <= 0.0f || x >= 1.0f) return 0.0;
  return 0.5 * double(-float(kPi) * sinf(float(kPi) * x)) / w;
}
__device__ __forceinline__ double smooth_ddist(double d, double rc, double w) {
  const double x = (d - (rc - w)) / w;
  if (x <= 0.0 || x >= 1.0) return 0.0;
  const double y = x * (1.0 - x);
  return -140.0 * y * y * y / w;
}
__device__ __forceinline__ double cutoff_ddist(double d, double rc, double w, int kind) {
  return kind == 0 ? bump_ddist(d, rc, w) : kind == 1 ? cosine_ddist(d, rc, w) : smooth_ddist(d, rc, w);
}

// The smooth cutoff factor of a distance (include/pet/cutoff.hpp:17-40): the
// transcendentals in float (the reference's CutT), the rest in double.
__device__ __forceinline__ double cutoff_value(double d, double rc, double w, int kind) {
  if (kind == 0) {
    const float x = float((d - (rc - w)) / w);
    if (x <= 0.0f) return 1.0;
    if (x >= 1.0f) return 0.0;
    return 0.5 * (1.0 + double(tanhf(1.0f / tanf(float(kPi) * x))));
  }
  if (kind == 1) {
    const float x = fminf(fmaxf(float((d - (rc - w)) / w), 0.0f), 1.0f);
    return 0.5 * (1.0 + double(cosf(float(kPi) * x)));
  }
  const double x = fmin(fmax((d - (rc - w)) / w, 0.0), 1.0);
  const double x4 = x * x * x * x;
  return 1.0 - x4 * (35.0 - 84.0 * x + 70.0 * x * x - 20.0 * x * x * x);
}

// An edge list's vectors, lengths and cutoff factors from positions
// (nef_vectors, src/device_geometry.cpp:335-345, then the factor of
// src/device_neighbors.cpp:214-260): v = r_j + shift . cell - r_i, a
// coincident pair's length 1e30 (it weighs nothing).
__global__ void edge_geometry_kernel(int E, const int* __restrict__ center, const int* __restrict__ neigh,
                                     const int* __restrict__ shift, const double* __restrict__ pos,
                                     const double* __restrict__ cell, double cutoff, double width, int kind,
                                     double* __restrict__ vec, double* __restrict__ dist, double* __restrict__ pcut,
                                     float* __restrict__ cut) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int i = center[e], j = neigh[e];
  const int s0 = shift ? shift[3 * e] : 0, s1 = shift ? shift[3 * e + 1] : 0, s2 = shift ? shift[3 * e + 2] : 0;
  double d2 = 0.0;
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const double sh = cell ? __dadd_rn(__dadd_rn(__dmul_rn(s0, cell[d]), __dmul_rn(s1, cell[3 + d])),
                                       __dmul_rn(s2, cell[6 + d]))
                           : 0.0;
    const double x = __dsub_rn(__dadd_rn(pos[3 * j + d], sh), pos[3 * i + d]);
    vec[3 * e + d] = x;
    d2 = __dadd_rn(d2, __dmul_rn(x, x));
  }
  const double r = d2 > 1e-24 ? sqrt(d2) : 1e30;
  dist[e] = r;
  pcut[e] = cutoff;
  cut[e] = float(cutoff_value(r, cutoff, width, kind));
}

__global__ void edge_grad_kernel(int nc, int E, const int* __restrict__ off, const int* __restrict__ center,
                                 const float* __restrict__ x4_adj, int64_t ldx, const float* __restrict__ cutoff_adj,
                                 const float* __restrict__ cf_seq_adj, int64_t ldca, const double* __restrict__ vec,
                                 const double* __restrict__ dist, const double* __restrict__ pcut, double width,
                                 int kind, double* __restrict__ grad) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= E) return;
  double* g = grad + 3 * int64_t(k);
  if (k >= off[nc]) {  // a capacity's dead row
    g[0] = g[1] = g[2] = 0.0;
    return;
  }
  const int n = center[k], m = k - off[n];
  const float* xa = x4_adj + int64_t(k) * ldx;
  // two fp32 values added in fp32, then widened (the reference's expression)
  const double cutoff_total = double((cutoff_adj ? cutoff_adj[k] : 0.0f) + cf_seq_adj[int64_t(n) * ldca + 1 + m]);
  const double dk = dist[k];
  const double dcut_dd = cutoff_ddist(dk, pcut[k], width, kind);
  const double dist_adj = double(xa[3]) + cutoff_total * dcut_dd;
  const double invd = dk > 0.0 ? 1.0 / dk : 0.0;
  const double* v = vec + 3 * int64_t(k);
#pragma unroll
  for (int c = 0; c < 3; ++c) g[c] = double(xa[c]) + dist_adj * v[c] * invd;
}

// One thread an atom, its edges in order: the reference's sums exactly.
__global__ void fold_kernel(int N, int nc, const int* __restrict__ off, const int* __restrict__ rev,
                            const double* __restrict__ vec, const double* __restrict__ grad, double scale,
                            double* __restrict__ forces, double* __restrict__ vir) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  double f[3] = {0.0, 0.0, 0.0}, w[9] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  const int k0 = i < nc ? off[i] : 0, k1 = i < nc ? off[i + 1] : 0;
  for (int k = k0; k < k1; ++k) {
    const double g0 = grad[3 * int64_t(k)], g1 = grad[3 * int64_t(k) + 1], g2 = grad[3 * int64_t(k) + 2];
    const double v0 = vec[3 * int64_t(k)], v1 = vec[3 * int64_t(k) + 1], v2 = vec[3 * int64_t(k) + 2];
    f[0] += g0, f[1] += g1, f[2] += g2;
    w[0] += v0 * g0, w[1] += v0 * g1, w[2] += v0 * g2;
    w[3] += v1 * g0, w[4] += v1 * g1, w[5] += v1 * g2;
    w[6] += v2 * g0, w[7] += v2 * g1, w[8] += v2 * g2;
    const int r = rev[k];
    if (r >= 0) {
      f[0] -= grad[3 * int64_t(r)], f[1] -= grad[3 * int64_t(r) + 1], f[2] -= grad[3 * int64_t(r) + 2];
    }
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) forces[3 * int64_t(i) + c] = scale * f[c];
  if (vir)
#pragma unroll
    for (int t = 0; t < 9; ++t) vir[9 * int64_t(i) + t] = scale * w[t];
}

// A wavefront per (structure, column): lane l sums atoms a0 + l, a0 + l + 64,
// ..., then a fixed butterfly over the lanes.
__global__ void __launch_bounds__(256) struct_sum_kernel(int NS, int width, const int* __restrict__ soff,
                                                         const double* __restrict__ x, double* __restrict__ out,
                                                         int acc) {
  const int item = blockIdx.x * 4 + int(threadIdx.x >> 6), l = threadIdx.x & 63;
  if (item >= NS * width) return;
  const int b = item / width, t = item - b * width;
  double s = 0.0;
  for (int a = soff[b] + l; a < soff[b + 1]; a += 64) s += x[int64_t(a) * width + t];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  if (l == 0) out[int64_t(b) * width + t] = acc ? out[int64_t(b) * width + t] + s : s;
}

}  // namespace pet_forces

using namespace pet_forces;

extern "C" {

int pet_edge_grad(int n_centres, int n_edges, const int* off, const int* center, const float* x4_adj, int64_t ldx,
                  const float* cutoff_adj, const float* cf_seq_adj, int64_t ldca, const double* vec,
                  const double* dist, const double* pcut, double width, int kind, double* grad, void* stream) {
  if (n_centres < 0 || n_edges < 0 || kind < 0 || kind > 2 || !(width > 0.0)) return PET_ATTN_EINVAL;
  if (n_edges == 0) return PET_ATTN_OK;
  if (!off || !center || !x4_adj || ldx < 4 || !cf_seq_adj || ldca < 1 || !vec || !dist || !pcut || !grad)
    return PET_ATTN_EINVAL;
  hipLaunchKernelGGL(edge_grad_kernel, dim3(unsigned((n_edges + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), n_centres, n_edges, off, center, x4_adj, ldx, cutoff_adj,
                     cf_seq_adj, ldca, vec, dist, pcut, width, kind, grad);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

int pet_fold_edge_gradients(int n_atoms, int n_centres, const int* off, const int* reverse, const double* vec,
                            const double* grad, double scale, double* forces, double* virial_atom, void* stream) {
  if (n_atoms < 0 || n_centres < 0 || n_centres > n_atoms) return PET_ATTN_EINVAL;
  if (n_atoms == 0) return PET_ATTN_OK;
  if (!forces || (n_centres > 0 && (!off || !reverse || !vec || !grad))) return PET_ATTN_EINVAL;
  hipLaunchKernelGGL(fold_kernel, dim3(unsigned((n_atoms + 127) / 128)), dim3(128), 0,
                     reinterpret_cast<hipStream_t>(stream), n_atoms, n_centres, off, reverse, vec, grad, scale, forces,
                     virial_atom);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

int pet_edge_geometry(int n_edges, const int* center, const int* neigh, const int* shift, const double* positions,
                      const double* cell, double cutoff, double width, int kind, double* vec, double* dist,
                      double* pcut, float* cut, void* stream) {
  if (n_edges < 0 || kind < 0 || kind > 2 || !(width > 0.0) || !(cutoff > 0.0)) return PET_ATTN_EINVAL;
  if (n_edges == 0) return PET_ATTN_OK;
  if (!center || !neigh || !positions || !vec || !dist || !pcut || !cut || (shift && !cell)) return PET_ATTN_EINVAL;
  hipLaunchKernelGGL(edge_geometry_kernel, dim3(unsigned((n_edges + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), n_edges, center, neigh, shift, positions, cell, cutoff,
                     width, kind, vec, dist, pcut, cut);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

int pet_sum_by_structure(int n_struct, int width, const int* soff, const double* x, double* out, int accumulate,
                         void* stream) {
  if (n_struct < 0 || width < 1) return PET_ATTN_EINVAL;
  if (n_struct == 0) return PET_ATTN_OK;
  if (!soff || !x || !out) return PET_ATTN_EINVAL;
  const int items = n_struct * width;
  hipLaunchKernelGGL(struct_sum_kernel, dim3(unsigned((items + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), n_struct, width, soff, x, out, accumulate);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}

}  // extern "C"
