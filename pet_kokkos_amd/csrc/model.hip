// The whole PET energy / forces evaluation on gfx950: the feedforward
// featurizer's forward and analytic backward around this library's attention
// (peterspackman/pet-kokkos src/feedforward.cpp:34-411), the readout and energy
// (src/model.cpp:656-780, src/ops.cpp:406-425) and forces_and_virial
// (src/forces.cpp:345-386) for a fixed cutoff.
//
// Every step outside the GEMMs is a kernel of this library: the attention
// (attention.hip), the norms (rows.hip), the edge term and folds (forces.hip)
// and, here, the gathers, compress.0's folded form, SiLU / SwiGLU and their
// backwards, the residual sums, the combination's concat and the readout. The
// dense layers go to rocBLAS fp32 (ops.hip's gemm_nt / gemm_nn, atomics off).
// The elementwise passes are HBM-bound: grid-stride loops over contiguous
// row-major buffers, one read and one write per value, residual sums fused
// into the pass that produces their operands.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/pet_model.h"

namespace pet_attn {
int gemm_nt(float* out, int64_t ldo, const float* in, int64_t ldi, const float* W, int M, int Nout, int K, float beta,
            hipStream_t st);
int gemm_nn(float* in_adj, int64_t ldi, const float* out_adj, int64_t ldo, const float* W, int M, int Nout, int K,
            float beta, hipStream_t st);
}  // namespace pet_attn
int pet_rows_norm_bwd_sink(int rows, int width, float* in_adj, int64_t lda, const float* out_adj, int64_t ldg,
                           const float* in, int64_t ldi, const float* weight, int ln, int n_node, float beta_node,
                           float beta_edge, const int* live_off, hipStream_t st);
// rows.hip: RMSNorm's row factors
int pet_rows_rms_inv(int rows, int width, const float* in, int64_t ldi, float* inv, hipStream_t st);
// gemm.hip: C = epilogue(A B^T)
int pet_gemm_nt_fused(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                      int64_t ldc, const float* row_scale, const float* bias, const float* cin, int64_t ldcin,
                      float beta, float* pre, int64_t ldpre, int act, hipStream_t st);
int pet_gemm_nt_split(int M, int N, int K, const float* A, int64_t lda, const void* Bs, float* C, int64_t ldc,
                      const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                      float* pre, int64_t ldpre, int act, hipStream_t st, void* scratch = nullptr,
                      size_t scratch_bytes = 0);

// gemm.hip: block pairs out of one product, into the next
int pet_gemm_nt_split_pairs(int M, int N, int K, const float* A, int64_t lda, const void* Bs, void* pout,
                            const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                            float* pre, int64_t ldpre, int act, hipStream_t st, void* scratch, size_t scratch_bytes,
                            int* kb);
int pet_gemm_nt_pp_to_blocks(int M, int N, int K, const void* Ap, const void* Bs, void* pout, const float* bias,
                             const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre, int act,
                             hipStream_t st, int* kb);
int pet_attn_bwd_xf_blocks(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const float* rs, const float* b,
                           const int* off, const float* dmerged, int64_t ldg, const float* merged, int64_t ldm,
                           const float* ml, const float* cf_seq, int64_t ldc, void* qpairs, float* cfh,
                           float* cf_seq_adj, int64_t ldca, hipStream_t st);
int pet_gemm_nt_pp_blocks(int M, int N, int K, const void* Ap, int kb, const void* Bs, float* C, int64_t ldc,
                          const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                          float* pre, int64_t ldpre, int act, hipStream_t st);

extern "C" int pet_linear_fused_smallk(int M, int N, int K, const float* A, int64_t lda, const void* Wpairs, float* C,
                                       int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                       int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream);
int pet_gemm_pair_weights(const float* W, int N, int K, int64_t ldw, bool transposed, void* out, hipStream_t st);

namespace pet_model_impl {

using pet_attn::gemm_nn;
using pet_attn::gemm_nt;

// ---- activations ---------------------------------------------------------------
//
// The SiLU / SwiGLU sigmoid of the dense layers is the hardware exp and
// reciprocal (the reference's fast_sigmoid on an AMD GPU in fp32,
// include/pet/kokkos.hpp:246-259); compress.0's SiLU takes the accurate one
// (src/ops.cpp:360 calls silu(), include/pet/kokkos.hpp:238-244).
__device__ __forceinline__ float sig_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float sig_exact(float x) { return 1.0f / (1.0f + expf(-x)); }

#define GRID_LOOP(i, n) \
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

// out[r, :] = table[idx[r], :]
__global__ void gather_rows_kernel(float* __restrict__ out, const float* __restrict__ table,
                                   const int* __restrict__ idx, int64_t R, int W) {
  GRID_LOOP(i, R * W) {
    const int64_t r = i / W;
    const int d = int(i - r * W);
    out[i] = table[int64_t(idx[r]) * W + d];
  }
}

// out[r, :] = b (or 0), the bias a GEMM then accumulates onto
__global__ void fill_rows_kernel(float* __restrict__ out, const float* __restrict__ b, int64_t R, int W) {
  GRID_LOOP(i, R * W) out[i] = b ? b[i % W] : 0.0f;
}

__global__ void fill0_kernel(float* __restrict__ x, int64_t n) {
  GRID_LOOP(i, n) x[i] = 0.0f;
}

// s = a + c (saved when s is non-null), then out = s + b: a residual sum and
// the bias of the GEMM that accumulates onto it.
__global__ void residual_kernel(float* __restrict__ s, float* __restrict__ out, const float* __restrict__ a,
                                const float* __restrict__ c, const float* __restrict__ b, int64_t R, int W) {
  GRID_LOOP(i, R * W) {
    const float v = a[i] + c[i];
    if (s) s[i] = v;
    out[i] = v + b[i % W];
  }
}

// x += b per row
__global__ void add_bias_kernel(float* __restrict__ x, const float* __restrict__ b, int64_t R, int W) {
  GRID_LOOP(i, R * W) x[i] += b[i % W];
}

// The dense layers before an activation run with beta 0 and no bias: their
// output z is kept as is (the saved pre-activation is z + b) and the
// activation passes, forward and backward, add the bias as they read it --
// one write and one read of the pre-activation fewer than a bias fill the
// GEMM accumulates onto. A layer on the split-product kernel instead takes the
// bias and the activation in the kernel's epilogue and saves z + b itself; its
// backward pass then gets a null bias (zero).

// out = silu(z + b), fast sigmoid (linear_silu, src/ops.cpp:54-76)
__global__ void silu_kernel(float* __restrict__ out, const float* __restrict__ z, const float* __restrict__ b,
                            int64_t R, int W) {
  GRID_LOOP(i, R * W) {
    const float v = z[i] + b[i % W];
    out[i] = v * sig_fast(v);
  }
}

// g *= silu'(pre + b) (silu_bwd, src/ops.cpp:78-101)
__global__ void silu_bwd_kernel(float* __restrict__ g, const float* __restrict__ pre, const float* __restrict__ b,
                                int64_t R, int W) {
  GRID_LOOP(i, R * W) {
    const float x = pre[i] + (b ? b[i % W] : 0.f), sg = sig_fast(x);
    g[i] *= sg * (1.0f + x * (1.0f - sg));
  }
}

// h[r, c] = v * sigmoid(g), (v, g) = pre[r, 2c .. 2c+1] + b[2c .. 2c+1]: pre's
// rows interleaved (v_j, g_j) (swiglu_in, src/ops.cpp:248-271)
__global__ void swiglu_kernel(float* __restrict__ h, const float2* __restrict__ pre, const float2* __restrict__ b,
                              int64_t R, int F) {
  GRID_LOOP(i, R * F) {
    const float2 p = pre[i], bb = b[i % F];
    const float v = p.x + bb.x, g = p.y + bb.y;
    h[i] = v * sig_fast(g);
  }
}

// pre_adj from h_adj (swiglu_bwd, src/ops.cpp:281-324)
__global__ void swiglu_bwd_kernel(float2* __restrict__ pre_adj, const float* __restrict__ h_adj,
                                  const float2* __restrict__ pre, const float2* __restrict__ b, int64_t R, int F) {
  GRID_LOOP(i, R * F) {
    const float2 p = pre[i], bb = b ? b[i % F] : make_float2(0.f, 0.f);
    const float v = p.x + bb.x, sg = sig_fast(p.y + bb.y), g = h_adj[i];
    pre_adj[i] = make_float2(g * sg, g * v * sg * (1.0f - sg));
  }
}

// compress.0 through its fold (compress_fwd, src/ops.cpp:326-371):
// z = [gemm] + b + tab[nsp] + wx (v, |v|); sav = z, out = silu(z), accurate sigmoid.
__global__ void compress_kernel(float* __restrict__ sav, float* __restrict__ out, int gemm,
                                const float* __restrict__ b, const float* __restrict__ tab,
                                const int* __restrict__ nsp, const float* __restrict__ wx,
                                const double* __restrict__ vec, const double* __restrict__ dist, int64_t E, int D) {
  GRID_LOOP(i, E * D) {
    const int64_t k = i / D;
    const int d = int(i - k * D);
    const float e0 = float(vec[3 * k]), e1 = float(vec[3 * k + 1]), e2 = float(vec[3 * k + 2]), e3 = float(dist[k]);
    const float* w = wx + 4 * d;
    const float z = (gemm ? out[i] : 0.0f) + b[d] + tab[int64_t(nsp[k]) * D + d] + w[0] * e0 + w[1] * e1 +
                    w[2] * e2 + w[3] * e3;
    sav[i] = z;
    out[i] = z * sig_exact(z);
  }
}

// compress_bwd's pass (src/ops.cpp:373-404): a wavefront a row, g *= silu'(pre)
// in place, and x4_adj[r] += the four sums g . wx[:, c] (a fixed butterfly).
__global__ void __launch_bounds__(256) compress_bwd_kernel(float* __restrict__ g, const float* __restrict__ pre,
                                                           const float* __restrict__ wx, float* __restrict__ x4_adj,
                                                           int E, int D) {
  const int r = blockIdx.x * 4 + int(threadIdx.x >> 6), l = threadIdx.x & 63;
  if (r >= E) return;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  float* gr = g + int64_t(r) * D;
  const float* pr = pre + int64_t(r) * D;
  for (int d = l; d < D; d += 64) {
    const float x = pr[d], sg = sig_fast(x);
    const float gd = gr[d] * (sg * (1.0f + x * (1.0f - sg)));
    gr[d] = gd;
    a0 += gd * wx[4 * d], a1 += gd * wx[4 * d + 1], a2 += gd * wx[4 * d + 2], a3 += gd * wx[4 * d + 3];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a0 += __shfl_xor(a0, o), a1 += __shfl_xor(a1, o);
    a2 += __shfl_xor(a2, o), a3 += __shfl_xor(a3, o);
  }
  if (l == 0) {
    float* x = x4_adj + 4 * int64_t(r);
    x[0] += a0, x[1] += a1, x[2] += a2, x[3] += a3;
  }
}

// The combination's input (src/feedforward.cpp:179-192): concat[k] = [oe(k) |
// oe(rev k) or 0], and input_edge += oe.
__global__ void concat_kernel(float* __restrict__ concat, float* __restrict__ ie, const float* __restrict__ oe,
                              const int* __restrict__ rev, int64_t E, int D) {
  GRID_LOOP(i, E * D) {
    const int64_t k = i / D;
    const int d = int(i - k * D), r = rev[k];
    const float v = oe[i];
    ie[i] += v;
    concat[k * 2 * D + d] = v;
    concat[k * 2 * D + D + d] = r >= 0 ? oe[int64_t(r) * D + d] : 0.0f;
  }
}

// edge_adj[k] = ie_adj[k] + ca[k, :D] + ca[rev k, D:] (bw_concat, src/feedforward.cpp:254-259)
__global__ void concat_bwd_kernel(float* __restrict__ edge_adj, const float* __restrict__ ie_adj,
                                  const float* __restrict__ ca, const int* __restrict__ rev, int64_t E, int D) {
  GRID_LOOP(i, E * D) {
    const int64_t k = i / D;
    const int d = int(i - k * D), r = rev[k];
    const float back = r >= 0 ? ca[int64_t(r) * 2 * D + D + d] : 0.0f;
    edge_adj[i] = ie_adj[i] + ca[k * 2 * D + d] + back;
  }
}

// net[n] (=, or += for acc, in fp32) node_pred[n] + the sum over n's edges
// of cut * edge_pred, in double and in edge order (readout_accumulate,
// src/ops.cpp:406-418).
__global__ void readout_kernel(float* __restrict__ net, const float* __restrict__ node_pred,
                               const float* __restrict__ edge_pred, const int* __restrict__ off,
                               const float* __restrict__ cut, int acc, int N) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  double s = node_pred[n];
  for (int k = off[n]; k < off[n + 1]; ++k) s += double(cut[k]) * double(edge_pred[k]);
  net[n] = acc ? float(double(net[n]) + s) : float(s);
}

// per_atom = scale * net + composition[species] (assemble_energy, src/ops.cpp:420-425)
__global__ void assemble_kernel(double* __restrict__ per_atom, const float* __restrict__ net,
                                const int* __restrict__ species, const double* __restrict__ comp, double scale,
                                int N) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < N) per_atom[n] = scale * double(net[n]) + comp[species[n]];
}

// The readout's adjoint seeds (readout_bwd, src/model.cpp:749-767): node_pred's
// is 1, edge_pred's the edge's cutoff factor, and cutoff_adj (+)= edge_pred.
__global__ void readout_seed_kernel(float* __restrict__ npa, float* __restrict__ epa, float* __restrict__ cutoff_adj,
                                    const float* __restrict__ cut, const float* __restrict__ epred, int acc, int N,
                                    int E) {
  GRID_LOOP(i, int64_t(N) + E) {
    if (i < N) {
      npa[i] = 1.0f;
    } else {
      const int64_t k = i - N;
      epa[k] = cut[k];
      cutoff_adj[k] = acc ? cutoff_adj[k] + epred[k] : epred[k];
    }
  }
}

// out = a + b per row
__global__ void bias_add_kernel(float* __restrict__ out, const float* __restrict__ a, const float* __restrict__ b,
                                int64_t R, int W) {
  GRID_LOOP(i, R * W) out[i] = a[i] + b[i % W];
}

__global__ void copy_kernel(float* __restrict__ out, const float* __restrict__ a, int64_t n) {
  GRID_LOOP(i, n) out[i] = a[i];
}

// out = s * a
__global__ void scale_kernel(float* __restrict__ out, const float* __restrict__ a, float s, int64_t n) {
  GRID_LOOP(i, n) out[i] = s * a[i];
}

// The residual featurizer's message passing (src/residual.cpp:122-131):
// input_edge[k] = 0.5 (input_edge[k] + out_edge[reverse k]), 0 for no reverse.
__global__ void message_kernel(float* __restrict__ ie, const float* __restrict__ oe, const int* __restrict__ rev,
                               int64_t E, int D) {
  GRID_LOOP(i, E * D) {
    const int64_t k = i / D;
    const int d = int(i - k * D), r = rev[k];
    ie[i] = 0.5f * (ie[i] + (r >= 0 ? oe[int64_t(r) * D + d] : 0.0f));
  }
}

// Its backward's reverse share (src/residual.cpp:183-190): efa[k] += 0.5 ie_adj[reverse k].
__global__ void message_bwd_kernel(float* __restrict__ efa, const float* __restrict__ ie_adj,
                                   const int* __restrict__ rev, int64_t E, int D) {
  GRID_LOOP(i, E * D) {
    const int64_t k = i / D;
    const int d = int(i - k * D), r = rev[k];
    efa[i] += r >= 0 ? 0.5f * ie_adj[int64_t(r) * D + d] : 0.0f;
  }
}

// ---- the same passes, 4 floats a thread ---------------------------------------
// For a width W with W / 4 dividing 256 (the model's widths) and 16-byte
// aligned rows: thread t of a workgroup keeps the column slice t % (W / 4) and
// steps over rows 256 / (W / 4) at a time, so every access is a 16-byte one and
// no index needs a 64-bit division. The arithmetic per value is the scalar
// kernels': the results are the same bits.
#define ROWS4_LOOP(r, c, R, W4)                  \
  const int c = int(threadIdx.x) % (W4);         \
  const int rpb_ = 256 / (W4);                   \
  for (int64_t r = int64_t(blockIdx.x) * rpb_ + int(threadIdx.x) / (W4); r < (R); r += int64_t(gridDim.x) * rpb_)

__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// The 16-byte forms of gather_rows_kernel, compress_kernel, concat_kernel
// and concat_bwd_kernel (rows of W4 float4 groups, rows4_ok): each thread
// takes whole groups, with the same arithmetic per element as the scalar
// forms below, and no 64-bit division an element.
__global__ void gather_rows4_kernel(float4* __restrict__ out, const float4* __restrict__ table,
                                    const int* __restrict__ idx, int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) out[r * W4 + c] = table[int64_t(idx[r]) * W4 + c];
}
__global__ void compress4_kernel(float4* __restrict__ sav, float4* __restrict__ out, int gemm,
                                 const float4* __restrict__ b, const float4* __restrict__ tab,
                                 const int* __restrict__ nsp, const float4* __restrict__ wx,
                                 const double* __restrict__ vec, const double* __restrict__ dist, int64_t E, int W4) {
  ROWS4_LOOP(k, c, E, W4) {
    const float e0 = float(vec[3 * k]), e1 = float(vec[3 * k + 1]), e2 = float(vec[3 * k + 2]), e3 = float(dist[k]);
    const int64_t i = k * W4 + c;
    const float4 g = gemm ? out[i] : make_float4(0.f, 0.f, 0.f, 0.f), bb = b[c], t = tab[int64_t(nsp[k]) * W4 + c];
    const float gv[4] = {g.x, g.y, g.z, g.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w}, tv[4] = {t.x, t.y, t.z, t.w};
    float z[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float4 w = wx[4 * c + u];  // column 4 c + u's four weights
      z[u] = (gemm ? gv[u] : 0.0f) + bv[u] + tv[u] + w.x * e0 + w.y * e1 + w.z * e2 + w.w * e3;
    }
    sav[i] = make_float4(z[0], z[1], z[2], z[3]);
    out[i] = make_float4(z[0] * sig_exact(z[0]), z[1] * sig_exact(z[1]), z[2] * sig_exact(z[2]),
                         z[3] * sig_exact(z[3]));
  }
}
__global__ void concat4_kernel(float4* __restrict__ concat, float4* __restrict__ ie, const float4* __restrict__ oe,
                               const int* __restrict__ rev, int64_t E, int W4) {
  ROWS4_LOOP(k, c, E, W4) {
    const int r = rev[k];
    const int64_t i = k * W4 + c;
    const float4 v = oe[i];
    ie[i] = add4(ie[i], v);
    concat[k * 2 * W4 + c] = v;
    concat[k * 2 * W4 + W4 + c] = r >= 0 ? oe[int64_t(r) * W4 + c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}
__global__ void concat_bwd4_kernel(float4* __restrict__ edge_adj, const float4* __restrict__ ie_adj,
                                   const float4* __restrict__ ca, const int* __restrict__ rev, int64_t E, int W4) {
  ROWS4_LOOP(k, c, E, W4) {
    const int r = rev[k];
    const float4 back = r >= 0 ? ca[int64_t(r) * 2 * W4 + W4 + c] : make_float4(0.f, 0.f, 0.f, 0.f);
    edge_adj[k * W4 + c] = add4(add4(ie_adj[k * W4 + c], ca[k * 2 * W4 + c]), back);
  }
}

__global__ void fill_rows4_kernel(float4* __restrict__ out, const float4* __restrict__ b, int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) out[r * W4 + c] = b ? b[c] : make_float4(0.f, 0.f, 0.f, 0.f);
}
__global__ void residual4_kernel(float4* __restrict__ s, float4* __restrict__ out, const float4* __restrict__ a,
                                 const float4* __restrict__ cc, const float4* __restrict__ b, int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) {
    const int64_t i = r * W4 + c;
    const float4 v = add4(a[i], cc[i]);
    if (s) s[i] = v;
    out[i] = add4(v, b[c]);
  }
}
__global__ void add_bias4_kernel(float4* __restrict__ x, const float4* __restrict__ b, int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) x[r * W4 + c] = add4(x[r * W4 + c], b[c]);
}
__global__ void bias_add4_kernel(float4* __restrict__ out, const float4* __restrict__ a, const float4* __restrict__ b,
                                 int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) out[r * W4 + c] = add4(a[r * W4 + c], b[c]);
}
__device__ __forceinline__ float silu1(float z, float b) {
  const float v = z + b;
  return v * sig_fast(v);
}
__global__ void silu4_kernel(float4* __restrict__ out, const float4* __restrict__ z, const float4* __restrict__ b,
                             int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) {
    const float4 x = z[r * W4 + c], bb = b[c];
    out[r * W4 + c] = make_float4(silu1(x.x, bb.x), silu1(x.y, bb.y), silu1(x.z, bb.z), silu1(x.w, bb.w));
  }
}
__device__ __forceinline__ float silu_bwd1(float g, float pre, float b) {
  const float x = pre + b, sg = sig_fast(x);
  return g * (sg * (1.0f + x * (1.0f - sg)));
}
template <bool HB>
__global__ void silu_bwd4_kernel(float4* __restrict__ g, const float4* __restrict__ pre, const float4* __restrict__ b,
                                 int64_t R, int W4) {
  ROWS4_LOOP(r, c, R, W4) {
    const int64_t i = r * W4 + c;
    const float4 gg = g[i], x = pre[i], bb = HB ? b[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    g[i] = make_float4(silu_bwd1(gg.x, x.x, bb.x), silu_bwd1(gg.y, x.y, bb.y), silu_bwd1(gg.z, x.z, bb.z),
                       silu_bwd1(gg.w, x.w, bb.w));
  }
}
// h has F4 float4 a row; pre and b hold (v, g) pairs, two float4 per h float4
__global__ void swiglu4_kernel(float4* __restrict__ h, const float4* __restrict__ pre, const float4* __restrict__ b,
                               int64_t R, int F4) {
  ROWS4_LOOP(r, c, R, F4) {
    const float4 p0 = pre[r * 2 * F4 + 2 * c], p1 = pre[r * 2 * F4 + 2 * c + 1], b0 = b[2 * c], b1 = b[2 * c + 1];
    h[r * F4 + c] = make_float4((p0.x + b0.x) * sig_fast(p0.y + b0.y), (p0.z + b0.z) * sig_fast(p0.w + b0.w),
                                (p1.x + b1.x) * sig_fast(p1.y + b1.y), (p1.z + b1.z) * sig_fast(p1.w + b1.w));
  }
}
__device__ __forceinline__ float2 swiglu_bwd1(float g, float pv, float pg, float bv, float bg) {
  const float v = pv + bv, sg = sig_fast(pg + bg);
  return make_float2(g * sg, g * v * sg * (1.0f - sg));
}
// HB false: pre holds its bias already (b unused)
template <bool HB>
__global__ void swiglu_bwd4_kernel(float4* __restrict__ pre_adj, const float4* __restrict__ h_adj,
                                   const float4* __restrict__ pre, const float4* __restrict__ b, int64_t R, int F4) {
  ROWS4_LOOP(r, c, R, F4) {
    const float4 g = h_adj[r * F4 + c], z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 p0 = pre[r * 2 * F4 + 2 * c], p1 = pre[r * 2 * F4 + 2 * c + 1];
    const float4 b0 = HB ? b[2 * c] : z4, b1 = HB ? b[2 * c + 1] : z4;
    const float2 a = swiglu_bwd1(g.x, p0.x, p0.y, b0.x, b0.y), bq = swiglu_bwd1(g.y, p0.z, p0.w, b0.z, b0.w);
    const float2 cq = swiglu_bwd1(g.z, p1.x, p1.y, b1.x, b1.y), d = swiglu_bwd1(g.w, p1.z, p1.w, b1.z, b1.w);
    pre_adj[r * 2 * F4 + 2 * c] = make_float4(a.x, a.y, bq.x, bq.y);
    pre_adj[r * 2 * F4 + 2 * c + 1] = make_float4(cq.x, cq.y, d.x, d.y);
  }
}
__global__ void copy4_kernel(float4* __restrict__ out, const float4* __restrict__ a, int64_t n4) {
  GRID_LOOP(i, n4) out[i] = a[i];
}
__global__ void scale4_kernel(float4* __restrict__ out, const float4* __restrict__ a, float s, int64_t n4) {
  GRID_LOOP(i, n4) {
    const float4 v = a[i];
    out[i] = make_float4(s * v.x, s * v.y, s * v.z, s * v.w);
  }
}
__global__ void fill04_kernel(float4* __restrict__ x, int64_t n4) {
  GRID_LOOP(i, n4) x[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// W / 4 divides 256 and every pointer (null allowed) is 16-byte aligned
inline bool rows4_ok(int W, std::initializer_list<const void*> ps) {
  if (W <= 0 || W % 4 || 256 % (W / 4)) return false;
  for (const void* p : ps)
    if (!al16(p)) return false;
  return true;
}
inline dim3 grid_rows4(int64_t R, int W4) {
  const int64_t b = (R + 256 / W4 - 1) / (256 / W4);
  return dim3(unsigned(b < 8192 ? (b > 0 ? b : 1) : 8192));
}
inline float4* v4(float* p) { return reinterpret_cast<float4*>(p); }
inline const float4* v4(const float* p) { return reinterpret_cast<const float4*>(p); }

inline dim3 grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return dim3(unsigned(b < 8192 ? (b > 0 ? b : 1) : 8192));
}

// ---- device memory -------------------------------------------------------------

// A bump arena over device blocks, kept across calls; mark / release reuse a
// scope's memory. After the first evaluation at a size nothing is allocated.
class Arena {
 public:
  ~Arena() {
    for (auto& b : blocks_) (void) hipFree(b.p);
  }
  struct Mark {
    size_t block, off;
  };
  Mark mark() const { return {cur_, off_}; }
  void release(Mark m) { cur_ = m.block, off_ = m.off; }
  void reset() { cur_ = 0, off_ = 0; }
  size_t bytes() const {
    size_t s = 0;
    for (auto& b : blocks_) s += b.size;
    return s;
  }
  // nullptr when the device is out of memory
  void* take(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes == 0) bytes = 256;
    while (cur_ < blocks_.size()) {
      if (off_ + bytes <= blocks_[cur_].size) {
        void* p = static_cast<char*>(blocks_[cur_].p) + off_;
        off_ += bytes;
        return p;
      }
      ++cur_, off_ = 0;
    }
    const size_t size = std::max(bytes, size_t(1) << 30);
    void* p = nullptr;
    if (hipMalloc(&p, size) != hipSuccess) return nullptr;
    blocks_.push_back({p, size});
    cur_ = blocks_.size() - 1;
    off_ = bytes;
    return p;
  }

 private:
  struct Block {
    void* p;
    size_t size;
  };
  std::vector<Block> blocks_;
  size_t cur_ = 0, off_ = 0;
};

struct Mat {
  float* p = nullptr;
  int rows = 0, cols = 0;
};

struct Error {
  int code;
};
inline void ok(int e) {
  if (e) throw Error{e};
}
inline void launched() {
  if (hipGetLastError() != hipSuccess) throw Error{PET_ATTN_ELAUNCH};
}

}  // namespace pet_model_impl

using namespace pet_model_impl;

struct pet_model {
  pet_model_hypers h{};
  int hd = 0, cw = 0, ew = 0;  // head_dim, center / edge MLP pre-activation widths
  int gemm_mode = 6;           // PET_OPT_MODEL_GEMM for the evaluation in progress
  bool blocks = true;          // PET_OPT_MODEL_PAIRS for the evaluation in progress
  int tier = 1;                // the memory tier of the last evaluation: 1 never, 2 wide
  std::unordered_map<std::string, Mat> m;
  std::unordered_map<const float*, const void*> split;  // a matrix's split-row copy (K a multiple of 32)
  std::unordered_map<const float*, const void*> psplit;  // its fp16 part rows at K <= 128 (the short-K kernel)
  // layers whose saved pre-activation holds its bias (made by the split-product
  // kernel's epilogue in the forward in progress), read by their backward
  std::unordered_map<std::string, bool> pre_biased;
  void* weights = nullptr;
  void* wsplit = nullptr;
  void* wpair = nullptr;
  double* comp = nullptr;
  // A's fp16 pairs for the split-product kernel's pairs-by-pairs path, a row
  // chunk at a time (null: that path is not taken)
  void* pairs = nullptr;
  static constexpr size_t kPairsBytes = size_t(512) << 20;
  Arena ws;

  ~pet_model() {
    if (weights || wsplit || wpair || comp || ws.bytes()) (void) hipDeviceSynchronize();
    if (weights) (void) hipFree(weights);
    if (wsplit) (void) hipFree(wsplit);
    if (wpair) (void) hipFree(wpair);
    if (comp) (void) hipFree(comp);
    if (pairs) (void) hipFree(pairs);
  }
  const Mat& w(const std::string& name) const {
    auto it = m.find(name);
    if (it == m.end()) throw Error{PET_MODEL_EMISSING};
    return it->second;
  }
  const float* p(const std::string& name) const { return w(name).p; }
  float* f(int64_t n) {
    void* q = ws.take(sizeof(float) * size_t(n));
    if (!q) throw Error{PET_MODEL_EMEMORY};
    return static_cast<float*>(q);
  }
};

namespace {

// Which forward dense layers take this library's fused GEMM (gemm.hip) instead
// of rocBLAS: 0 none (the default), 1 all, 2 those with at most 4096 rows.
// Measured on MI355X (C2 / C2-residual / C5 energy+forces, ms): 3.45 / 2.67 /
// 281 with rocBLAS, 3.50 / 2.68 / 281 with mode 2, 3.96 / 3.00 / 311 with mode
// 1: its main loop reaches 72% of the fp32 matrix peak at K = 1024 where
// rocBLAS reaches 90%. The option PET_OPT_MODEL_GEMM selects (md.gemm_mode,
// read once at the start of each evaluation).
bool own_gemm(const pet_model& md, int M, int K) {
  return K % 16 == 0 && (md.gemm_mode == 1 || (md.gemm_mode == 2 && M <= 4096));
}

// out[M, N] = in W^T + beta out, W a model matrix [N, K]: rocBLAS fp32, or
// this library's kernels where W has a copy in their form and in is 16-byte
// aligned rows. By PET_OPT_MODEL_GEMM: 6 (the default) the split-product
// kernel for the large products (M N K >= 2^32), the short-K kernel
// (pet_linear_fused_smallk: the weights exact in three fp16 parts, A's rows
// as fp16 pairs, five part products) for the K <= 128 products with a bias or
// activation and N >= 64, rocBLAS for the rest; 4 as 6 without the short-K
// kernel; 5 every product on this library's kernels -- the short-K kernel for
// K at most 128, the split-product kernel above -- so that no result depends
// on how many rows come with it and every bias and activation rides in an
// epilogue; 3 the split-product kernel for every product; 0 rocBLAS only.
// Measured on MI355X (energy+forces, ms): C2 2.585 / 1.92 (residual) with
// mode 6, 2.80 / 2.07 with mode 4 (no C2 product is large), 2.89 / 1.95 with
// mode 5, 3.59 / 2.40 with mode 3; C5 171 with mode 4, 170 with mode 5.
// Energies from the float64 oracle, C2 / residual: mode 6 3.0e-7 / 3.8e-7,
// mode 4 0.7e-7 / 4.2e-7, mode 5 1.5e-7 / 8.3e-7 (the float32 oracle 3.3e-7 /
// 4.2e-7). The narrow products (N < 64: the readout's) stay off the short-K
// kernel: its matrix instruction truncates each product toward zero below the
// result's last place, and with a fixed weight vector and mostly positive
// inputs those truncations share a sign on every atom and add up over a
// structure (C2-residual 5.7e-7 with them on it).
// The kernel a product takes (null: rocBLAS): the copy of W it reads and
// whether it is the short-K kernel.
struct Sel {
  const void* p = nullptr;
  bool sk = false;
  explicit operator bool() const { return p != nullptr; }
};
// fuse: the call has a bias or an activation for the epilogue (mode 6 takes
// the short-K kernel for those products at K <= 128 and N >= 64, where it
// saves a pass).
Sel split_for(const pet_model& md, const float* in, int64_t ldi, const float* W, int M, int N, int K,
              bool fuse = false) {
  const int mode = md.gemm_mode;
  const bool big = double(M) * N * K >= 4294967296.0;
  if (ldi % 4 || (reinterpret_cast<uintptr_t>(in) & 15)) return {};
  if ((mode == 5 || (mode == 6 && fuse && N >= 64)) && K <= 128 && K % 32 == 0) {
    auto it = md.psplit.find(W);
    if (it != md.psplit.end()) return {it->second, true};
  }
  if (mode == 3 || mode == 5 || ((mode == 4 || mode == 6) && big)) {
    auto it = md.split.find(W);
    if (it != md.split.end()) return {it->second, false};
  }
  return {};
}
// C = epilogue(in W^T) on the kernel sel names
int own_nt(const pet_model& md, const Sel& sel, int M, int N, int K, const float* in, int64_t ldi, float* C,
           int64_t ldc, const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
           float* pre, int64_t ldpre, int act, hipStream_t st) {
  if (sel.sk)
    return pet_linear_fused_smallk(M, N, K, in, ldi, sel.p, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre,
                                   act, st);
  return pet_gemm_nt_split(M, N, K, in, ldi, sel.p, C, ldc, row_scale, bias, cin, ldcin, beta, pre, ldpre, act, st,
                           md.pairs, md.pairs ? md.kPairsBytes : 0);
}
int gemm_w(const pet_model& md, float* out, int64_t ldo, const float* in, int64_t ldi, const float* W, int M, int N,
           int K, float beta, hipStream_t st) {
  if (const Sel sp = split_for(md, in, ldi, W, M, N, K))
    return own_nt(md, sp, M, N, K, in, ldi, out, ldo, nullptr, nullptr, beta != 0.f ? out : nullptr, ldo, beta,
                  nullptr, 0, 0, st);
  return gemm_nt(out, ldo, in, ldi, W, M, N, K, beta, st);
}

// out[M, Nout] = in W^T + b (b may be null)
void linear(pet_model& md, float* out, const float* in, int M, int K, const std::string& key, hipStream_t st,
            bool bias = true) {
  const Mat& W = md.w(key + ".weight");
  if (W.cols != K) throw Error{PET_MODEL_ESHAPE};
  if (M == 0) return;
  const float* b = bias ? md.p(key + ".bias") : nullptr;
  if (own_gemm(md, M, K)) {
    ok(pet_gemm_nt_fused(M, W.rows, K, in, K, W.p, K, out, W.rows, nullptr, b, nullptr, 0, 0.f, nullptr, 0, 0, st));
    return;
  }
  if (const Sel sp = split_for(md, in, K, W.p, M, W.rows, K, b != nullptr)) {  // the bias in the epilogue
    ok(own_nt(md, sp, M, W.rows, K, in, K, out, W.rows, nullptr, b, nullptr, 0, 0.f, nullptr, 0, 0, st));
    return;
  }
  if (rows4_ok(W.rows, {out, b}))
    hipLaunchKernelGGL(fill_rows4_kernel, grid_rows4(M, W.rows / 4), dim3(256), 0, st, v4(out), v4(b), int64_t(M),
                       W.rows / 4);
  else
    hipLaunchKernelGGL(fill_rows_kernel, grid_for(int64_t(M) * W.rows), dim3(256), 0, st, out, b, int64_t(M), W.rows);
  launched();
  ok(gemm_w(md, out, W.rows, in, K, W.p, M, W.rows, K, 1.0f, st));
}
// out += in W^T (the caller has put residual + bias in out)
void linear_acc(pet_model& md, float* out, const float* in, int M, int K, const std::string& key, hipStream_t st) {
  const Mat& W = md.w(key + ".weight");
  if (W.cols != K) throw Error{PET_MODEL_ESHAPE};
  if (M == 0) return;
  if (own_gemm(md, M, K)) {
    ok(pet_gemm_nt_fused(M, W.rows, K, in, K, W.p, K, out, W.rows, nullptr, nullptr, out, W.rows, 1.f, nullptr, 0, 0,
                         st));
    return;
  }
  ok(gemm_w(md, out, W.rows, in, K, W.p, M, W.rows, K, 1.0f, st));
}
void add_bias_pass(float* x, const float* b, int64_t R, int W, hipStream_t st);
// out += in W^T + b: the bias in the split-product kernel's epilogue where the
// layer takes that kernel, else a bias pass before linear_acc
void linear_acc_bias(pet_model& md, float* out, const float* in, int M, int K, const std::string& key,
                     hipStream_t st) {
  const Mat& W = md.w(key + ".weight");
  if (W.cols != K) throw Error{PET_MODEL_ESHAPE};
  if (M == 0) return;
  if (const Sel sp = own_gemm(md, M, K) ? Sel{} : split_for(md, in, K, W.p, M, W.rows, K, true)) {
    ok(own_nt(md, sp, M, W.rows, K, in, K, out, W.rows, nullptr, md.p(key + ".bias"), out, W.rows, 1.f, nullptr, 0, 0,
              st));
    return;
  }
  add_bias_pass(out, md.p(key + ".bias"), int64_t(M), W.rows, st);
  linear_acc(md, out, in, M, K, key, st);
}
// in_adj[M, K] = out_adj W + beta in_adj
void linear_bwd(pet_model& md, float* in_adj, const float* out_adj, int M, const std::string& key, float beta,
                hipStream_t st) {
  const Mat& WT = md.w(key + ".weight^T");  // [K, Nout]: out_adj W = out_adj (W^T)^T
  if (M) ok(gemm_w(md, in_adj, WT.rows, out_adj, WT.cols, WT.p, M, WT.rows, WT.cols, beta, st));
}
// The backward of linear_act's activation fused into the product before it:
// out = act'(z) * (adj W) (act 1 SiLU: out [M, Nout]; 2 SwiGLU: out [M, 2 Nout]
// from the (value, gate) pairs of z), adj W the input adjoint of layer
// key_out, z the saved pre-activation of layer key_act -- one split-product
// GEMM with the activation's backward in its epilogue (the same product and
// the same per-element arithmetic as linear_bwd then silu_bwd / swiglu_bwd),
// where that layer takes the split kernel. True when fused.
const float* pass_bias(const pet_model& md, const std::string& key);
bool linear_bwd_act(pet_model& md, float* out, const float* adj, int M, const std::string& key_out, const float* z,
                    const std::string& key_act, int act, hipStream_t st) {
  const Mat& WT = md.w(key_out + ".weight^T");
  const Sel sp = M ? split_for(md, adj, WT.cols, WT.p, M, WT.rows, WT.cols, true) : Sel{};
  if (!sp) return false;
  const int64_t w = act == 2 ? 2 * int64_t(WT.rows) : WT.rows;
  ok(own_nt(md, sp, M, WT.rows, WT.cols, adj, WT.cols, out, w, nullptr, pass_bias(md, key_act), z, w, 0.f, nullptr, 0,
            act == 2 ? 4 : 3, st));
  return true;
}
// z[M, Nout] = in W^T, no bias: the pre-activation an activation pass reads with its bias
void linear_pre(pet_model& md, float* z, const float* in, int M, int K, const std::string& key, hipStream_t st) {
  const Mat& W = md.w(key + ".weight");
  if (W.cols != K) throw Error{PET_MODEL_ESHAPE};
  if (M == 0) return;
  if (own_gemm(md, M, K)) {
    ok(pet_gemm_nt_fused(M, W.rows, K, in, K, W.p, K, z, W.rows, nullptr, nullptr, nullptr, 0, 0.f, nullptr, 0, 0,
                         st));
    return;
  }
  ok(gemm_w(md, z, W.rows, in, K, W.p, M, W.rows, K, 0.0f, st));
}
// z = in W^T + b and out = act(z) (act 1 SiLU, 2 SwiGLU) as one split-product
// GEMM with the bias and the activation in its epilogue, where the layer takes
// that kernel (then z holds its bias, recorded for the backward); else
// linear_pre and the activation pass. True when fused.
// Whether linear_act fuses the layer (then out must be a buffer other than in).
bool act_fuses(const pet_model& md, const float* in, int M, int K, const std::string& key) {
  const Mat& W = md.w(key + ".weight");
  return !own_gemm(md, M, K) && bool(split_for(md, in, K, W.p, M, W.rows, K, true));
}
bool linear_act(pet_model& md, float* out, float* z, const float* in, int M, int K, const std::string& key, int act,
                hipStream_t st) {
  const Mat& W = md.w(key + ".weight");
  if (W.cols != K) throw Error{PET_MODEL_ESHAPE};
  // (out must not be the GEMM's input: other workgroups still read its rows)
  const Sel sp = own_gemm(md, M, K) || out == in ? Sel{} : split_for(md, in, K, W.p, M, W.rows, K, true);
  md.pre_biased[key] = bool(sp);
  if (!sp || M == 0) return false;
  ok(own_nt(md, sp, M, W.rows, K, in, K, out, act == 2 ? W.rows / 2 : W.rows, nullptr, md.p(key + ".bias"), nullptr, 0,
            0.f, z, W.rows, act, st));
  return true;
}
// ---- block pairs between two products ----------------------------------------
//
// Where an activation (SiLU, SwiGLU) or its adjoint is read by the next
// product alone, and both products take the split kernel's pairs-by-pairs
// form, the first writes it as block pairs (pet_gemm_nt_split_pairs: fp16
// pairs scaled per row and 128-column tile of the product) and the second
// reads them as its A (pet_gemm_nt_pp_blocks), in place of an fp32 round trip
// and a split pass (C5 energy+forces on MI355X: see pet_gemm_nt_split_pairs).
// The pre-activation the backward reads is the same bits either way.
int out_cols(int N, int act) { return act == 2 ? N / 2 : act == 4 ? 2 * N : N; }
struct Blocks {
  void* p = nullptr;
  int kb = 0, cols = 0;
};
// the split copy of W when the product (M x N x K) takes the pairs-by-pairs form
const void* pp_split(const pet_model& md, const Mat& W, int M, int N, int K) {
  const int mode = md.gemm_mode;
  const bool big = double(M) * N * K >= 4294967296.0;
  if (!(mode == 3 || mode == 5 || ((mode == 4 || mode == 6) && big)) || (mode == 5 && K <= 128)) return nullptr;
  if (K < 256 || K % 32 || N < 512) return nullptr;
  auto it = md.split.find(W.p);
  return it == md.split.end() ? nullptr : it->second;
}
// Whether out = act(in Wa^T ...) (M x Wa.rows x K) and the product out Wb^T
// chain as block pairs (Wa, Wb as the products read them: row-major [N, K]).
bool chains(const pet_model& md, int M, int K, const Mat& Wa, int act, const Mat& Wb) {
  if (!md.blocks || !md.pairs || M <= 0) return false;
  const int N = Wa.rows, no = out_cols(N, act), kb = out_cols(128, act);
  if (N % 128 || no % kb || no / kb > 32 || Wb.cols != no) return false;
  return pp_split(md, Wa, M, N, K) && pp_split(md, Wb, M, Wb.rows, no);
}
// the producer: act(in W^T + bias) as block pairs (act 1 / 2, pre kept and
// biased), or (act 3 / 4) the adjoint adj W^T through the saved pre-activation z
Blocks blocks_out(pet_model& md, const float* in, int M, int K, const Mat& W, int act, const float* bias,
                  const float* z, float* pre, hipStream_t st) {
  Blocks b;
  b.cols = out_cols(W.rows, act);
  b.p = md.f(int64_t(M) * b.cols + int64_t(M) * (b.cols / 32) + 4);
  const int64_t ldz = act == 4 ? 2 * int64_t(W.rows) : W.rows;
  ok(pet_gemm_nt_split_pairs(M, W.rows, K, in, K, pp_split(md, W, M, W.rows, K), b.p, nullptr, bias, z,
                             z ? ldz : 0, 0.f, pre, pre ? W.rows : 0, act, st, md.pairs, md.kPairsBytes, &b.kb));
  return b;
}
// the producer from the norm of rows `in` (width K: RMSNorm, or LayerNorm with
// a bias) made directly as pair rows (pet_norm_rows_pairs: the bits the split
// pass gives for the fp32 norm), act 1 / 2 with the pre-activation kept
// (the pair rows into `room` where it holds them: room_floats floats no one
// reads any more)
Blocks blocks_out_normed(pet_model& md, const float* in, int M, int K, const std::string& norm_key, bool ln,
                         const Mat& W, int act, const float* bias, float* pre, hipStream_t st, float* room = nullptr,
                         int64_t room_floats = 0) {
  const int64_t apf = int64_t(M) * K + M + 4;
  void* ap = room && room_floats >= apf ? static_cast<void*>(room) : md.f(apf);
  ok(pet_norm_rows_pairs(M, K, ap, in, K, md.p(norm_key + ".weight"), ln ? md.p(norm_key + ".bias") : nullptr, st));
  Blocks b;
  b.cols = out_cols(W.rows, act);
  b.p = md.f(int64_t(M) * b.cols + int64_t(M) * (b.cols / 32) + 4);
  ok(pet_gemm_nt_pp_to_blocks(M, W.rows, K, ap, pp_split(md, W, M, W.rows, K), b.p, bias, nullptr, 0, 0.f, pre,
                              pre ? W.rows : 0, act, st, &b.kb));
  return b;
}
// the consumer: C = B W^T + bias + beta cin
void blocks_in(pet_model& md, float* C, const Blocks& b, int M, const Mat& W, const float* bias, const float* cin,
               float beta, hipStream_t st) {
  ok(pet_gemm_nt_pp_blocks(M, W.rows, b.cols, b.p, b.kb, pp_split(md, W, M, W.rows, b.cols), C, W.rows, nullptr,
                           bias, cin, cin ? W.rows : 0, beta, nullptr, 0, 0, st));
}

// the bias the activation passes add to a saved pre-activation: none where the
// forward's epilogue put it in already
const float* pass_bias(const pet_model& md, const std::string& key) {
  auto it = md.pre_biased.find(key);
  return it != md.pre_biased.end() && it->second ? nullptr : md.p(key + ".bias");
}
// out = silu(z + b) of linear_pre's z under `key`
void silu(pet_model& md, float* out, const float* z, int64_t R, const std::string& key, hipStream_t st) {
  const Mat& b = md.w(key + ".bias");
  if (R == 0) return;
  if (rows4_ok(b.rows, {out, z, b.p}))
    hipLaunchKernelGGL(silu4_kernel, grid_rows4(R, b.rows / 4), dim3(256), 0, st, v4(out), v4(z), v4(b.p), R,
                       b.rows / 4);
  else
    hipLaunchKernelGGL(silu_kernel, grid_for(R * b.rows), dim3(256), 0, st, out, z, b.p, R, b.rows);
  launched();
}
void silu_bwd(pet_model& md, float* g, const float* z, int64_t R, const std::string& key, hipStream_t st) {
  const Mat& b = md.w(key + ".bias");
  const float* bp = pass_bias(md, key);
  if (R == 0) return;
  if (rows4_ok(b.rows, {g, z, b.p}))
    hipLaunchKernelGGL(bp ? silu_bwd4_kernel<true> : silu_bwd4_kernel<false>, grid_rows4(R, b.rows / 4), dim3(256),
                       0, st, v4(g), v4(z), v4(bp), R, b.rows / 4);
  else
    hipLaunchKernelGGL(silu_bwd_kernel, grid_for(R * b.rows), dim3(256), 0, st, g, z, bp, R, b.rows);
  launched();
}
// h = swiglu(z + b) of linear_pre's z under `key` (a .w_in)
void swiglu(pet_model& md, float* h, const float* z, int64_t R, const std::string& key, hipStream_t st) {
  const Mat& b = md.w(key + ".bias");
  if (R == 0) return;
  if (b.rows % 2 == 0 && rows4_ok(b.rows / 2, {h, z, b.p}))
    hipLaunchKernelGGL(swiglu4_kernel, grid_rows4(R, b.rows / 8), dim3(256), 0, st, v4(h), v4(z), v4(b.p), R,
                       b.rows / 8);
  else
    hipLaunchKernelGGL(swiglu_kernel, grid_for(R * b.rows / 2), dim3(256), 0, st, h,
                       reinterpret_cast<const float2*>(z), reinterpret_cast<const float2*>(b.p), R, b.rows / 2);
  launched();
}
void swiglu_bwd(pet_model& md, float* z_adj, const float* h_adj, const float* z, int64_t R, const std::string& key,
                hipStream_t st) {
  const Mat& b = md.w(key + ".bias");
  const float* bp = pass_bias(md, key);
  if (R == 0) return;
  if (b.rows % 2 == 0 && rows4_ok(b.rows / 2, {z_adj, h_adj, z, b.p}))
    hipLaunchKernelGGL(bp ? swiglu_bwd4_kernel<true> : swiglu_bwd4_kernel<false>, grid_rows4(R, b.rows / 8),
                       dim3(256), 0, st, v4(z_adj), v4(h_adj), v4(z), v4(bp), R, b.rows / 8);
  else
    hipLaunchKernelGGL(swiglu_bwd_kernel, grid_for(R * b.rows / 2), dim3(256), 0, st,
                       reinterpret_cast<float2*>(z_adj), h_adj, reinterpret_cast<const float2*>(z),
                       reinterpret_cast<const float2*>(bp), R, b.rows / 2);
  launched();
}
// The elementwise passes: the float4 kernels where the width and alignment allow.
// out[r, :] = table[idx[r], :] for R rows of W floats (16 bytes a thread where the rows allow)
void gather_rows(float* out, const float* table, const int* idx, int64_t R, int W, hipStream_t st) {
  if (rows4_ok(W, {out, table}))
    hipLaunchKernelGGL(gather_rows4_kernel, grid_rows4(R, W / 4), dim3(256), 0, st, v4(out), v4(table), idx, R, W / 4);
  else
    hipLaunchKernelGGL(gather_rows_kernel, grid_for(R * W), dim3(256), 0, st, out, table, idx, R, W);
}
void residual_pass(float* sv, float* out, const float* a, const float* c, const float* b, int64_t R, int W,
                   hipStream_t st) {
  if (R == 0) return;
  if (rows4_ok(W, {sv, out, a, c, b}))
    hipLaunchKernelGGL(residual4_kernel, grid_rows4(R, W / 4), dim3(256), 0, st, v4(sv), v4(out), v4(a), v4(c), v4(b),
                       R, W / 4);
  else
    hipLaunchKernelGGL(residual_kernel, grid_for(R * W), dim3(256), 0, st, sv, out, a, c, b, R, W);
  launched();
}
void add_bias_pass(float* x, const float* b, int64_t R, int W, hipStream_t st) {
  if (R == 0) return;
  if (rows4_ok(W, {x, b}))
    hipLaunchKernelGGL(add_bias4_kernel, grid_rows4(R, W / 4), dim3(256), 0, st, v4(x), v4(b), R, W / 4);
  else
    hipLaunchKernelGGL(add_bias_kernel, grid_for(R * W), dim3(256), 0, st, x, b, R, W);
  launched();
}
void bias_add_pass(float* out, const float* a, const float* b, int64_t R, int W, hipStream_t st) {
  if (R == 0) return;
  if (rows4_ok(W, {out, a, b}))
    hipLaunchKernelGGL(bias_add4_kernel, grid_rows4(R, W / 4), dim3(256), 0, st, v4(out), v4(a), v4(b), R, W / 4);
  else
    hipLaunchKernelGGL(bias_add_kernel, grid_for(R * W), dim3(256), 0, st, out, a, b, R, W);
  launched();
}
void copy_pass(float* out, const float* a, int64_t n, hipStream_t st) {
  if (n == 0) return;
  if (n % 4 == 0 && al16(out) && al16(a))
    hipLaunchKernelGGL(copy4_kernel, grid_for(n / 4), dim3(256), 0, st, v4(out), v4(a), n / 4);
  else
    hipLaunchKernelGGL(copy_kernel, grid_for(n), dim3(256), 0, st, out, a, n);
  launched();
}
void scale_pass(float* out, const float* a, float sc, int64_t n, hipStream_t st) {
  if (n == 0) return;
  if (n % 4 == 0 && al16(out) && al16(a))
    hipLaunchKernelGGL(scale4_kernel, grid_for(n / 4), dim3(256), 0, st, v4(out), v4(a), sc, n / 4);
  else
    hipLaunchKernelGGL(scale_kernel, grid_for(n), dim3(256), 0, st, out, a, sc, n);
  launched();
}
void norm(pet_model& md, float* out, const float* in, int R, int W, const std::string& key, bool ln, hipStream_t st) {
  ok(pet_norm_rows(R, W, out, W, in, W, md.p(key + ".weight"), ln ? md.p(key + ".bias") : nullptr, st));
}
void fill0(float* x, int64_t n, hipStream_t st) {
  if (n % 4 == 0 && al16(x))
    hipLaunchKernelGGL(fill04_kernel, grid_for(n / 4), dim3(256), 0, st, v4(x), n / 4);
  else
    hipLaunchKernelGGL(fill0_kernel, grid_for(n), dim3(256), 0, st, x, n);
  launched();
}

// What one GNN layer keeps for its backward (the reference's LayerSaves,
// include/pet/model.hpp:183-198): under the "never" tier every block's wide
// activations too (qkv, the edge MLP's pre-activation pre_e); under "wide"
// those two are null and the backward remakes them.
struct Block {
  float *tok, *inv, *qkv, *merged, *ml, *eps, *node_res, *pre_c, *pre_e;
};
struct Layer {
  float *cpre, *concat, *cph;
  std::vector<Block> b;
};

struct Pass {
  pet_model& md;
  const pet_model_edges& e;
  hipStream_t st;
  int N, E, T, S, D, Dn, Dh, A, G;
  pet_attn_shape sh{};
  float* cf_seq = nullptr;
  bool wide = false;  // the "wide" memory tier (recompute_tier)
  int chunk = 0;      // edge rows of an edge-MLP chunk under it

  Pass(pet_model& m, const pet_model_edges& ed, hipStream_t s) : md(m), e(ed), st(s) {
    N = e.n_atoms, E = e.n_edges, T = N + E, S = e.max_neighbors + 1;
    D = md.h.d_pet, Dn = md.h.d_node, Dh = md.h.d_head, A = md.h.num_attention_layers, G = md.h.num_gnn_layers;
    // the reference's chunk (PetModel::edge_chunk_rows, src/model.cpp:812-817):
    // an eighth of the edges and at least 64k rows, where the products run at
    // full speed and (at or above 2^32 multiply-adds) on the split-product
    // kernel, whose rows do not depend on how many there are
    chunk = std::max(65536, (E + 7) / 8);
    sh.n_atoms = N, sh.n_rows = T, sh.slots = S, sh.heads = md.h.num_heads, sh.head_dim = md.hd, sh.dead = 0;
    sh.scale = pet_attn_scale(md.hd, md.h.attention_temperature);
  }
  std::string g(int L) const { return "gnn_layers." + std::to_string(L); }
  std::string t(int L, int a) const { return g(L) + ".trans.layers." + std::to_string(a); }

  // The edge MLP's SwiGLU of rows of its normed input en (rows x D) into he
  // (rows x ew / 2), its pre-activation into a temporary the caller's scope
  // releases, which it returns: the forward's product and activation, so
  // the backward of the "wide" tier remakes the same bits.
  float* edge_pre(float* he, const float* en, int rows, const std::string& tl) {
    float* pre = md.f(int64_t(rows) * md.ew);
    if (!linear_act(md, he, pre, en, rows, D, tl + ".mlp.w_in", 2, st)) {
      linear_pre(md, pre, en, rows, D, tl + ".mlp.w_in", st);
      swiglu(md, he, pre, rows, tl + ".mlp.w_in", st);
    }
    return pre;
  }

  // One GNN layer forward (ff_layer, src/feedforward.cpp:34-198; under the
  // "wide" tier without its qkv and edge pre-activation saves).
  void layer_fwd(int L, float*& node, float* input_edge, Layer& sv) {
    sv.cpre = md.f(int64_t(E) * D);
    sv.b.resize(A);
    for (int a = 0; a < A; ++a) sv.b[a].tok = md.f(int64_t(T) * D);
    float* out_edge = md.f(int64_t(E) * D);
    compress_fwd(L, input_edge, sv.cpre, sv.b[0].tok + int64_t(N) * D);
    float* node_cur = node;
    const float* edge_cur = sv.b[0].tok + int64_t(N) * D;
    for (int a = 0; a < A; ++a) {
      const std::string tl = t(L, a);
      Block& b = sv.b[a];
      b.qkv = wide ? nullptr : md.f(int64_t(T) * 3 * D), b.merged = md.f(int64_t(T) * D);
      b.ml = md.f(int64_t(N) * md.h.num_heads * S * 2);
      b.eps = md.f(int64_t(E) * D), b.node_res = md.f(int64_t(N) * Dn), b.inv = md.f(T);
      b.pre_c = md.f(int64_t(N) * md.cw), b.pre_e = wide ? nullptr : md.f(int64_t(E) * md.ew);
      float* node_next = md.f(int64_t(N) * Dn);
      float* edge_next = a + 1 < A ? sv.b[a + 1].tok + int64_t(N) * D : out_edge;
      auto scope = md.ws.mark();
      linear(md, b.tok, node_cur, N, Dn, tl + ".center_contraction", st);
      // the fused QKV projection: qkv = tok (W_in diag(norm weight))^T, the
      // attention applying 1/rms and the bias as it loads it
      ok(pet_rows_rms_inv(T, D, b.tok, D, b.inv, st));
      float* qkv = wide ? md.f(int64_t(T) * 3 * D) : b.qkv;
      linear_pre(md, qkv, b.tok, T, D, tl + ".attention.input_linear@fold", st);
      ok(pet_attn_fwd_xf(&sh, qkv, 3 * D, b.inv, md.p(tl + ".attention.input_linear.bias"), e.off, cf_seq, S,
                         b.merged, D, b.ml, st));
      float* attn_out = md.f(int64_t(T) * D);
      const Mat& wi = md.w(tl + ".mlp.w_in.weight");
      const Mat& wo = md.w(tl + ".mlp.w_out.weight");
      // Where the output linear takes the split kernel and the edge MLP chains
      // as block pairs, the edge rows' residual rides in epilogues: the output
      // linear's edge rows go straight to eps = merged W^T + b + edge_cur (the
      // same bits as the residual pass's), and the edge MLP's last product adds
      // its bias and eps itself, so edge_next is never filled by a pass of its
      // own. The node rows and the edge rows take the kernel the whole matrix
      // would (a row's results do not depend on the others).
      const Mat& wout = md.w(tl + ".attention.output_linear.weight");
      const Sel so = split_for(md, b.merged, D, wout.p, T, D, D);
      const bool fuse_res = E > 0 && bool(so) && chains(md, wide ? std::min(chunk, E) : E, D, wi, 2, wo);
      if (fuse_res) {
        const float* bo = md.p(tl + ".attention.output_linear.bias");
        if (N) ok(own_nt(md, so, N, D, D, b.merged, D, attn_out, D, nullptr, bo, nullptr, 0, 0.f, nullptr, 0, 0, st));
        ok(own_nt(md, so, E, D, D, b.merged + int64_t(N) * D, D, b.eps, D, nullptr, bo, edge_cur, D, 1.f, nullptr, 0, 0,
                  st));
      } else {
        linear(md, attn_out, b.merged, T, D, tl + ".attention.output_linear", st);
      }
      float* node_exp = md.f(int64_t(N) * Dn);
      linear(md, node_exp, attn_out, N, D, tl + ".center_expansion", st);
      // eps = attention's edge rows + edge_cur; edge_next = eps + mlp's output bias
      if (E && !fuse_res) {
        residual_pass(b.eps, edge_next, attn_out + int64_t(N) * D, edge_cur, md.p(tl + ".mlp.w_out.bias"),
                      int64_t(E), D, st);
      }
      if (N) {
        residual_pass(b.node_res, node_next, node_cur, node_exp, md.p(tl + ".center_mlp.w_out.bias"), int64_t(N),
                      Dn, st);
      }
      // node_next += center_mlp(norm(node_res)); edge_next += mlp(norm(eps))
      float* nn = node_exp;  // consumed
      norm(md, nn, b.node_res, N, Dn, tl + ".norm_center_features", false, st);
      float* hc = md.f(int64_t(N) * md.cw / 2);
      if (!linear_act(md, hc, b.pre_c, nn, N, Dn, tl + ".center_mlp.w_in", 2, st)) {
        linear_pre(md, b.pre_c, nn, N, Dn, tl + ".center_mlp.w_in", st);
        swiglu(md, hc, b.pre_c, N, tl + ".center_mlp.w_in", st);
      }
      linear_acc(md, node_next, hc, N, md.cw / 2, tl + ".center_mlp.w_out", st);
      float* en = attn_out;  // consumed: its edge rows were read by the residual pass (or never written)
      // edge_next += SwiGLU(en W_in^T + b_in) W_out^T over rows [e0, e0 + rows),
      // the pre-activation into pre: the SwiGLU output as block pairs where the
      // two products chain so
      // (en = norm(eps) rows into enr, or as pair rows straight from the norm)
      // (attn_out is dead by then: all of it is room for the norm's pair rows
      // of the whole edge MLP)
      auto edge_mlp = [&](int e0, int rows, float* enr, float* pre) {
        float* out = edge_next + int64_t(e0) * D;
        const float* epsr = b.eps + int64_t(e0) * D;
        if (chains(md, rows, D, wi, 2, wo)) {
          md.pre_biased[tl + ".mlp.w_in"] = true;
          const bool all = rows == E;
          const Blocks hb = blocks_out_normed(md, epsr, rows, D, tl + ".norm_mlp", false, wi, 2,
                                             md.p(tl + ".mlp.w_in.bias"), pre, st, all ? attn_out : nullptr,
                                             all ? int64_t(T) * D : 0);
          if (fuse_res)  // edge_next = h W^T + b + eps
            blocks_in(md, out, hb, rows, wo, md.p(tl + ".mlp.w_out.bias"), epsr, 1.f, st);
          else  // edge_next (eps + b already) += h W^T
            blocks_in(md, out, hb, rows, wo, nullptr, out, 1.f, st);
          return;
        }
        if (fuse_res) bias_add_pass(out, epsr, md.p(tl + ".mlp.w_out.bias"), rows, D, st);  // edge_next = eps + b
        norm(md, enr, epsr, rows, D, tl + ".norm_mlp", false, st);
        float* he = md.f(int64_t(rows) * md.ew / 2);
        if (!linear_act(md, he, pre, enr, rows, D, tl + ".mlp.w_in", 2, st)) {
          linear_pre(md, pre, enr, rows, D, tl + ".mlp.w_in", st);
          swiglu(md, he, pre, rows, tl + ".mlp.w_in", st);
        }
        linear_acc(md, out, he, rows, md.ew / 2, tl + ".mlp.w_out", st);
      };
      if (!wide) {
        edge_mlp(0, E, en, b.pre_e);
      } else {  // a chunk of edge rows at a time, its pre-activation a temporary
        for (int e0 = 0; e0 < E; e0 += chunk) {
          const int rows = std::min(chunk, E - e0);
          auto sc = md.ws.mark();
          edge_mlp(e0, rows, en + int64_t(e0) * D, md.f(int64_t(rows) * md.ew));
          md.ws.release(sc);
        }
      }
      md.ws.release(scope);
      node_cur = node_next;
      edge_cur = edge_next;
    }
    node = node_cur;
    // input_edge += out_edge + comb_mlp(layernorm([out_edge | out_edge(rev)]))
    const std::string ls = std::to_string(L);
    sv.concat = md.f(int64_t(E) * 2 * D), sv.cph = md.f(int64_t(E) * 2 * D);
    auto scope = md.ws.mark();
    if (E) {
      if (rows4_ok(D, {sv.concat, input_edge, out_edge}))
        hipLaunchKernelGGL(concat4_kernel, grid_rows4(E, D / 4), dim3(256), 0, st, v4(sv.concat), v4(input_edge),
                           v4(out_edge), e.reverse, int64_t(E), D / 4);
      else
        hipLaunchKernelGGL(concat_kernel, grid_for(int64_t(E) * D), dim3(256), 0, st, sv.concat, input_edge, out_edge,
                           e.reverse, int64_t(E), D);
      launched();
    }
    const std::string c0 = "combination_mlps." + ls + ".0", c2 = "combination_mlps." + ls + ".2";
    if (chains(md, E, 2 * D, md.w(c0 + ".weight"), 1, md.w(c2 + ".weight"))) {
      // the norm as pair rows, the SiLU's output as block pairs
      md.pre_biased[c0] = true;
      const Blocks cb = blocks_out_normed(md, sv.concat, E, 2 * D, "combination_norms." + ls, true,
                                          md.w(c0 + ".weight"), 1, md.p(c0 + ".bias"), sv.cph, st);
      blocks_in(md, input_edge, cb, E, md.w(c2 + ".weight"), md.p(c2 + ".bias"), input_edge, 1.f, st);
      md.ws.release(scope);
      return;
    }
    float* cn = md.f(int64_t(E) * 2 * D);
    norm(md, cn, sv.concat, E, 2 * D, "combination_norms." + ls, true, st);
    // the SiLU's output: in place, or a buffer of its own for the fused GEMM
    // (which cannot write its input)
    float* ca = act_fuses(md, cn, E, 2 * D, c0) ? md.f(int64_t(E) * 2 * D) : cn;
    if (!linear_act(md, ca, sv.cph, cn, E, 2 * D, c0, 1, st)) {
      linear_pre(md, sv.cph, cn, E, 2 * D, c0, st);
      silu(md, ca, sv.cph, E, c0, st);
    }
    linear_acc_bias(md, input_edge, ca, E, 2 * D, c2, st);
    md.ws.release(scope);
  }

  // Its backward (ff_layer_bwd, src/feedforward.cpp:200-336): node_adj and
  // ie_adj from the layer's outputs' adjoints to its inputs', in place; x4_adj
  // and cf_seq_adj accumulate.
  void layer_bwd(int L, const Layer& sv, float* node_adj, float* ie_adj, float* x4_adj, float* cf_seq_adj) {
    const std::string ls = std::to_string(L);
    auto scope = md.ws.mark();
    float* tok_adj = md.f(int64_t(T) * D);
    float* edge_adj = tok_adj + int64_t(N) * D;
    {
      auto s2 = md.ws.mark();
      float* cn_adj = md.f(int64_t(E) * 2 * D);
      const std::string c0 = "combination_mlps." + ls + ".0", c2 = "combination_mlps." + ls + ".2";
      const Mat& c2t = md.w(c2 + ".weight^T");
      float* ca;  // the norm's input adjoint, in the buffer of the SiLU adjoint, consumed by then
      if (chains(md, E, c2t.cols, c2t, 3, md.w(c0 + ".weight^T"))) {  // the SiLU adjoint as block pairs
        const Blocks cb = blocks_out(md, ie_adj, E, c2t.cols, c2t, 3, pass_bias(md, c0), sv.cph, nullptr, st);
        blocks_in(md, cn_adj, cb, E, md.w(c0 + ".weight^T"), nullptr, nullptr, 0.f, st);
        ca = static_cast<float*>(cb.p);  // E (2D + 2D / 32) floats
      } else {
        float* cph_adj = md.f(int64_t(E) * 2 * D);
        if (!linear_bwd_act(md, cph_adj, ie_adj, E, c2, sv.cph, c0, 1, st)) {
          linear_bwd(md, cph_adj, ie_adj, E, c2, 0.0f, st);
          silu_bwd(md, cph_adj, sv.cph, E, c0, st);
        }
        linear_bwd(md, cn_adj, cph_adj, E, c0, 0.0f, st);
        ca = cph_adj;
      }
      ok(pet_norm_rows_bwd(E, 2 * D, ca, 2 * D, 0.0f, cn_adj, 2 * D, sv.concat, 2 * D,
                           md.p("combination_norms." + ls + ".weight"), 1, st));
      if (E) {
        if (rows4_ok(D, {edge_adj, ie_adj, ca}))
          hipLaunchKernelGGL(concat_bwd4_kernel, grid_rows4(E, D / 4), dim3(256), 0, st, v4(edge_adj), v4(ie_adj),
                             v4(ca), e.reverse, int64_t(E), D / 4);
        else
          hipLaunchKernelGGL(concat_bwd_kernel, grid_for(int64_t(E) * D), dim3(256), 0, st, edge_adj, ie_adj, ca,
                             e.reverse, int64_t(E), D);
        launched();
      }
      md.ws.release(s2);
    }
    for (int a = A - 1; a >= 0; --a) {
      const std::string tl = t(L, a);
      const Block& b = sv.b[a];
      auto s2 = md.ws.mark();
      {  // the two MLPs: edge_adj and node_adj become eps's and node_res's
        // the edge MLP over edge rows [e0, e0 + rows): all of them, or (wide) a
        // chunk at a time with its normed input and pre-activation remade
        auto edge_mlp_bwd = [&](int e0, int rows, const float* pre) {
          float* ea = edge_adj + int64_t(e0) * D;
          float* en_adj = md.f(int64_t(rows) * D);
          const Mat& wot = md.w(tl + ".mlp.w_out.weight^T");
          if (chains(md, rows, wot.cols, wot, 4, md.w(tl + ".mlp.w_in.weight^T"))) {  // SwiGLU's adjoint as block pairs
            const Blocks pb = blocks_out(md, ea, rows, wot.cols, wot, 4, pass_bias(md, tl + ".mlp.w_in"), pre, nullptr,
                                         st);
            blocks_in(md, en_adj, pb, rows, md.w(tl + ".mlp.w_in.weight^T"), nullptr, nullptr, 0.f, st);
          } else {
            float* h_adj = md.f(int64_t(rows) * md.ew / 2);
            float* pre_adj = md.f(int64_t(rows) * md.ew);
            if (!linear_bwd_act(md, pre_adj, ea, rows, tl + ".mlp.w_out", pre, tl + ".mlp.w_in", 2, st)) {
              linear_bwd(md, h_adj, ea, rows, tl + ".mlp.w_out", 0.0f, st);
              swiglu_bwd(md, pre_adj, h_adj, pre, rows, tl + ".mlp.w_in", st);
            }
            linear_bwd(md, en_adj, pre_adj, rows, tl + ".mlp.w_in", 0.0f, st);
          }
          ok(pet_norm_rows_bwd(rows, D, ea, D, 1.0f, en_adj, D, b.eps + int64_t(e0) * D, D,
                               md.p(tl + ".norm_mlp.weight"), 0, st));
        };
        if (!wide) {
          edge_mlp_bwd(0, E, b.pre_e);
        } else {
          for (int e0 = 0; e0 < E; e0 += chunk) {
            const int rows = std::min(chunk, E - e0);
            auto sc = md.ws.mark();
            float* en = md.f(int64_t(rows) * D);
            norm(md, en, b.eps + int64_t(e0) * D, rows, D, tl + ".norm_mlp", false, st);
            float* he = md.f(int64_t(rows) * md.ew / 2);
            const float* pre = edge_pre(he, en, rows, tl);
            edge_mlp_bwd(e0, rows, pre);
            md.ws.release(sc);
          }
        }
        float* hc_adj = md.f(int64_t(N) * md.cw / 2);
        float* prec_adj = md.f(int64_t(N) * md.cw);
        float* cn_adj = md.f(int64_t(N) * Dn);
        if (!linear_bwd_act(md, prec_adj, node_adj, N, tl + ".center_mlp.w_out", b.pre_c, tl + ".center_mlp.w_in", 2,
                            st)) {
          linear_bwd(md, hc_adj, node_adj, N, tl + ".center_mlp.w_out", 0.0f, st);
          swiglu_bwd(md, prec_adj, hc_adj, b.pre_c, N, tl + ".center_mlp.w_in", st);
        }
        linear_bwd(md, cn_adj, prec_adj, N, tl + ".center_mlp.w_in", 0.0f, st);
        ok(pet_norm_rows_bwd(N, Dn, node_adj, Dn, 1.0f, cn_adj, Dn, b.node_res, Dn,
                             md.p(tl + ".norm_center_features.weight"), 0, st));
      }
      md.ws.release(s2);
      // The attention: its output's adjoint is the expansion's input adjoint on
      // the atom rows and eps's (edge_adj, in place) on the edge rows.
      linear_bwd(md, tok_adj, node_adj, N, tl + ".center_expansion", 0.0f, st);
      float* dmerged = md.f(int64_t(T) * D);
      // (with room for the inverse scales of qkv_adj as block pairs)
      float* qkv_adj = md.f(int64_t(T) * (3 * D + 3 * md.h.num_heads) + 4);
      float* cfh = md.f(int64_t(N) * md.h.num_heads * S);
      float* in_adj = dmerged;
      linear_bwd(md, dmerged, tok_adj, T, tl + ".attention.output_linear", 0.0f, st);
      float* qkv = b.qkv;
      if (wide) {  // remade as the forward made it
        qkv = md.f(int64_t(T) * 3 * D);
        linear_pre(md, qkv, b.tok, T, D, tl + ".attention.input_linear@fold", st);
      }
      // qkv_adj as block pairs straight into the input adjoint's product where
      // that product takes the pairs-by-pairs form (block pairs); else fp32
      const Mat& wit = md.w(tl + ".attention.input_linear.weight^T");
      const void* wsp = md.blocks && md.pairs ? pp_split(md, wit, T, wit.rows, wit.cols) : nullptr;
      const int rc = wsp ? pet_attn_bwd_xf_blocks(&sh, qkv, 3 * D, b.inv, md.p(tl + ".attention.input_linear.bias"),
                                                  e.off, dmerged, D, b.merged, D, b.ml, cf_seq, S, qkv_adj, cfh,
                                                  cf_seq_adj, S, st)
                         : int(PET_ATTN_ESLOTS);
      if (rc == PET_ATTN_OK) {
        ok(pet_gemm_nt_pp_blocks(T, wit.rows, wit.cols, qkv_adj, md.hd, wsp, in_adj, wit.rows, nullptr, nullptr,
                                 nullptr, 0, 0.f, nullptr, 0, 0, st));
      } else {
        if (rc != PET_ATTN_ESLOTS) ok(rc);
        ok(pet_attn_bwd_xf(&sh, qkv, 3 * D, b.inv, md.p(tl + ".attention.input_linear.bias"), e.off, dmerged, D,
                           b.merged, D, b.ml, cf_seq, S, qkv_adj, 3 * D, cfh, cf_seq_adj, S, st));
        linear_bwd(md, in_adj, qkv_adj, T, tl + ".attention.input_linear", 0.0f, st);
      }
      // through the norm: atom rows set (input_node's adjoint), edge rows onto edge_adj
      ok(pet_rows_norm_bwd_sink(T, D, tok_adj, D, in_adj, D, b.tok, D, md.p(tl + ".norm_attention.weight"), 0, N,
                                0.0f, 1.0f, e.off, st));
      linear_bwd(md, node_adj, tok_adj, N, tl + ".center_contraction", 1.0f, st);
      md.ws.release(s2);
    }
    // edge_adj is et's: back through compress.2 and compress.0's fold
    compress_bwd(L, edge_adj, sv.cpre, x4_adj, ie_adj);
    md.ws.release(scope);
  }

  // One read-out (src/model.cpp:656-691): two SiLU layers and a last linear a
  // side, from node rows (width Dn) and edge rows (width D); net (fp32) = its
  // node prediction + sum of cut * edge predictions, or += for acc
  // (readout_accumulate, src/ops.cpp:406-418). Keeps the pre-activations.
  struct Readout {
    float *nh0, *nh1, *eh0, *eh1, *npred, *epred;
  };
  Readout readout_fwd(int i, const float* node_rows, const float* edge_rows, float* net, bool acc) {
    const std::string si = std::to_string(i), nh = "node_heads.energy." + si, eh = "edge_heads.energy." + si;
    Readout r{md.f(int64_t(N) * Dh), md.f(int64_t(N) * Dh), md.f(int64_t(E) * Dh), md.f(int64_t(E) * Dh), md.f(N),
              md.f(E)};
    auto scope = md.ws.mark();
    const int64_t rows = std::max<int64_t>(int64_t(N), int64_t(E)) * Dh;
    // a second buffer only where a fused layer would otherwise write its input
    float* x = md.f(rows);
    float* y = act_fuses(md, x, N, Dh, nh + ".2") || act_fuses(md, x, E, Dh, eh + ".2") ? md.f(rows) : x;
    auto layer = [&](float* out, float* z, const float* in, int M, int K, const std::string& key) {
      if (!linear_act(md, out, z, in, M, K, key, 1, st)) {
        linear_pre(md, z, in, M, K, key, st);
        silu(md, out, z, M, key, st);
      }
    };
    layer(x, r.nh0, node_rows, N, Dn, nh + ".0");
    layer(y, r.nh1, x, N, Dh, nh + ".2");
    linear(md, r.npred, y, N, Dh, "node_last_layers.energy." + si + ".energy___0", st);
    layer(x, r.eh0, edge_rows, E, D, eh + ".0");
    layer(y, r.eh1, x, E, Dh, eh + ".2");
    linear(md, r.epred, y, E, Dh, "edge_last_layers.energy." + si + ".energy___0", st);
    md.ws.release(scope);
    if (N) {
      hipLaunchKernelGGL(readout_kernel, dim3(unsigned((N + 255) / 256)), dim3(256), 0, st, net, r.npred, r.epred,
                         e.off, e.cut, acc ? 1 : 0, N);
      launched();
    }
    return r;
  }
  // Its backward (readout_bwd, src/model.cpp:749-780): node_adj [N, Dn] and
  // edge_adj [E, D] written, cutoff_adj written (or added to, acc).
  void readout_bwd(int i, const Readout& r, float* node_adj, float* edge_adj, float* cutoff_adj, bool acc) {
    const std::string si = std::to_string(i), nh = "node_heads.energy." + si, eh = "edge_heads.energy." + si;
    auto scope = md.ws.mark();
    float *npa = md.f(N), *epa = md.f(E), *a1 = md.f(std::max<int64_t>(N, E) * Dh),
          *a0 = md.f(std::max<int64_t>(N, E) * Dh);
    if (N + E) {
      hipLaunchKernelGGL(readout_seed_kernel, grid_for(int64_t(N) + E), dim3(256), 0, st, npa, epa, cutoff_adj,
                         e.cut, r.epred, acc ? 1 : 0, N, E);
      launched();
    }
    // each SiLU's backward in the epilogue of the product before it where it can be
    auto bwd_act = [&](float* out, const float* adj, int M, const std::string& ko, const float* z,
                       const std::string& ka) {
      if (!linear_bwd_act(md, out, adj, M, ko, z, ka, 1, st)) {
        linear_bwd(md, out, adj, M, ko, 0.0f, st);
        silu_bwd(md, out, z, M, ka, st);
      }
    };
    bwd_act(a1, npa, N, "node_last_layers.energy." + si + ".energy___0", r.nh1, nh + ".2");
    bwd_act(a0, a1, N, nh + ".2", r.nh0, nh + ".0");
    linear_bwd(md, node_adj, a0, N, nh + ".0", 0.0f, st);
    bwd_act(a1, epa, E, "edge_last_layers.energy." + si + ".energy___0", r.eh1, eh + ".2");
    bwd_act(a0, a1, E, eh + ".2", r.eh0, eh + ".0");
    linear_bwd(md, edge_adj, a0, E, eh + ".0", 0.0f, st);
    md.ws.release(scope);
  }

  // compress.0 (folded) and compress.2 of layer L into et [E, D] (ld D); the
  // pre-activation kept in cpre.
  void compress_fwd(int L, const float* input_edge, float* cpre, float* et) {
    const std::string c0 = g(L) + ".compress.0";
    auto scope = md.ws.mark();
    float* cact = md.f(int64_t(E) * D);
    if (L > 0) ok(gemm_w(md, cact, D, input_edge, D, md.p(c0 + "@in"), E, D, D, 0.0f, st));
    if (E) {
      const float *cb = md.p(c0 + "@b"), *ctab = md.p(c0 + "@tab"), *cx4 = md.p(c0 + "@x4");
      if (rows4_ok(D, {cpre, cact, cb, ctab, cx4}))
        hipLaunchKernelGGL(compress4_kernel, grid_rows4(E, D / 4), dim3(256), 0, st, v4(cpre), v4(cact), L > 0 ? 1 : 0,
                           v4(cb), v4(ctab), e.neigh_species, v4(cx4), e.vec, e.dist, int64_t(E), D / 4);
      else
        hipLaunchKernelGGL(compress_kernel, grid_for(int64_t(E) * D), dim3(256), 0, st, cpre, cact, L > 0 ? 1 : 0, cb,
                           ctab, e.neigh_species, cx4, e.vec, e.dist, int64_t(E), D);
      launched();
    }
    linear(md, et, cact, E, D, g(L) + ".compress.2", st);
    md.ws.release(scope);
  }
  // Its backward from et_adj (compress_bwd, src/ops.cpp:373-404): x4_adj +=,
  // and past layer 0 ie_adj += the input_edge block's share.
  void compress_bwd(int L, const float* et_adj, const float* cpre, float* x4_adj, float* ie_adj) {
    const std::string c0 = g(L) + ".compress.0";
    auto scope = md.ws.mark();
    float* ga = md.f(int64_t(E) * D);
    linear_bwd(md, ga, et_adj, E, g(L) + ".compress.2", 0.0f, st);
    if (E) {
      hipLaunchKernelGGL(compress_bwd_kernel, dim3(unsigned((E + 3) / 4)), dim3(256), 0, st, ga, cpre,
                         md.p(c0 + "@x4"), x4_adj, E, D);
      launched();
    }
    if (L > 0 && E) ok(gemm_w(md, ie_adj, D, ga, D, md.p(c0 + "@in^T"), E, D, D, 1.0f, st));
    md.ws.release(scope);
  }

  // What one residual GNN layer keeps (the reference's ResidualSaves, every
  // wide activation kept): per block qkv, merged, ml, s1 = attention + tokens,
  // s2 = mlp + LayerNorm(s1), and the MLP's pre-activation.
  struct RBlock {
    float *qkv, *merged, *ml, *s1, *s2, *pre;
  };
  struct RLayer {
    float *tokens, *cpre;
    std::vector<RBlock> b;
    Readout ro;
  };

  // residual_layer (src/residual.cpp:13-60): tokens = [node_L ; et], then A
  // PostLN blocks tokens = LN(s2), s2 = LN(s1) + mlp(LN(s1)), s1 = tokens +
  // attention(tokens), in place.
  void residual_layer_fwd(int L, const float* input_edge, RLayer& sv) {
    sv.tokens = md.f(int64_t(T) * D), sv.cpre = md.f(int64_t(E) * D);
    if (N) {
      gather_rows(sv.tokens, md.p("node_embedders." + std::to_string(L) + ".weight"), e.species, N, D, st);
      launched();
    }
    compress_fwd(L, input_edge, sv.cpre, sv.tokens + int64_t(N) * D);
    sv.b.resize(A);
    const int F = md.ew;
    for (int a = 0; a < A; ++a) {
      const std::string tl = t(L, a);
      RBlock& b = sv.b[a];
      b.qkv = md.f(int64_t(T) * 3 * D), b.merged = md.f(int64_t(T) * D), b.ml = md.f(int64_t(N) * md.h.num_heads * S * 2);
      b.s1 = md.f(int64_t(T) * D), b.s2 = md.f(int64_t(T) * D), b.pre = md.f(int64_t(T) * F);
      auto scope = md.ws.mark();
      // qkv without its bias, which the attention adds as it loads it
      linear_pre(md, b.qkv, sv.tokens, T, D, tl + ".attention.input_linear", st);
      ok(pet_attn_fwd_xf(&sh, b.qkv, 3 * D, nullptr, md.p(tl + ".attention.input_linear.bias"), e.off, cf_seq, S,
                         b.merged, D, b.ml, st));
      // s1 = tokens + b_out, then += merged W_out^T
      bias_add_pass(b.s1, sv.tokens, md.p(tl + ".attention.output_linear.bias"), int64_t(T), D, st);
      linear_acc(md, b.s1, b.merged, T, D, tl + ".attention.output_linear", st);
      float* tok_a = md.f(int64_t(T) * D);
      norm(md, tok_a, b.s1, T, D, tl + ".norm_attention", true, st);
      // s2 = tok_a + b_out, then += silu(tok_a W_in^T + b_in) W_out^T
      float* hm = md.f(int64_t(T) * F);
      if (!linear_act(md, hm, b.pre, tok_a, T, D, tl + ".mlp.w_in", 1, st)) {
        linear_pre(md, b.pre, tok_a, T, D, tl + ".mlp.w_in", st);
        silu(md, hm, b.pre, T, tl + ".mlp.w_in", st);
      }
      bias_add_pass(b.s2, tok_a, md.p(tl + ".mlp.w_out.bias"), int64_t(T), D, st);
      linear_acc(md, b.s2, hm, T, F, tl + ".mlp.w_out", st);
      norm(md, sv.tokens, b.s2, T, D, tl + ".norm_mlp", true, st);
      md.ws.release(scope);
    }
  }

  // Its backward (residual_pass, src/residual.cpp:180-226): tokens_adj is the
  // layer's output tokens' adjoint (overwritten); returns the adjoint of the
  // tokens the layer began with.
  float* residual_layer_bwd(int L, const RLayer& sv, float* tokens_adj, float* cf_seq_adj) {
    const int F = md.ew;
    for (int a = A - 1; a >= 0; --a) {
      const std::string tl = t(L, a);
      const RBlock& b = sv.b[a];
      auto scope = md.ws.mark();
      // tokens = LN(s2): s2_adj; tok_a_adj = s2_adj (the residual) + the MLP's input adjoint
      float* s2_adj = md.f(int64_t(T) * D);
      float* tok_a_adj = md.f(int64_t(T) * D);
      ok(pet_norm_rows_bwd(T, D, s2_adj, D, 0.0f, tokens_adj, D, b.s2, D, md.p(tl + ".norm_mlp.weight"), 1, st));
      copy_pass(tok_a_adj, s2_adj, int64_t(T) * D, st);
      float* h_adj = md.f(int64_t(T) * F);
      if (!linear_bwd_act(md, h_adj, s2_adj, T, tl + ".mlp.w_out", b.pre, tl + ".mlp.w_in", 1, st)) {
        linear_bwd(md, h_adj, s2_adj, T, tl + ".mlp.w_out", 0.0f, st);
        silu_bwd(md, h_adj, b.pre, T, tl + ".mlp.w_in", st);
      }
      linear_bwd(md, tok_a_adj, h_adj, T, tl + ".mlp.w_in", 1.0f, st);
      // tok_a = LN(s1): s1_adj into tokens_adj (consumed); the attention's input
      // adjoint then accumulates onto it (s1 = tokens + attention(tokens))
      ok(pet_norm_rows_bwd(T, D, tokens_adj, D, 0.0f, tok_a_adj, D, b.s1, D, md.p(tl + ".norm_attention.weight"), 1,
                           st));
      float* dmerged = md.f(int64_t(T) * D);
      float* qkv_adj = md.f(int64_t(T) * 3 * D);
      float* cfh = md.f(int64_t(N) * md.h.num_heads * S);
      linear_bwd(md, dmerged, tokens_adj, T, tl + ".attention.output_linear", 0.0f, st);
      ok(pet_attn_bwd_xf(&sh, b.qkv, 3 * D, nullptr, md.p(tl + ".attention.input_linear.bias"), e.off, dmerged, D,
                         b.merged, D, b.ml, cf_seq, S, qkv_adj, 3 * D, cfh, cf_seq_adj, S, st));
      linear_bwd(md, tokens_adj, qkv_adj, T, tl + ".attention.input_linear", 1.0f, st);
      md.ws.release(scope);
    }
    return tokens_adj;
  }

  void run(bool grad, double* energy, double* per_atom_out, double* forces, double* virial, double* edge_grad_out) {
    md.ws.reset();
    cf_seq = md.f(int64_t(N) * S);
    ok(pet_attn_cf_seq(&sh, e.off, e.cut, cf_seq, S, st));
    float* input_edge = md.f(int64_t(E) * D);
    if (E) {
      gather_rows(input_edge, md.p("edge_embedder.weight"), e.neigh_species, E, D, st);
      launched();
    }
    float* net = md.f(N);
    const bool residual = md.h.featurizer == 1;
    std::vector<Layer> sv(residual ? 0 : G);
    std::vector<RLayer> rv(residual ? G : 0);
    Readout ro{};
    if (residual) {
      // residual_pass (src/residual.cpp:62-133): a read-out after every layer,
      // then input_edge = (input_edge + out_edge(reverse)) / 2
      for (int L = 0; L < G; ++L) {
        residual_layer_fwd(L, input_edge, rv[L]);
        const float* edge_out = rv[L].tokens + int64_t(N) * D;
        rv[L].ro = readout_fwd(L, rv[L].tokens, edge_out, net, L > 0);
        if (L + 1 < G && E) {
          hipLaunchKernelGGL(message_kernel, grid_for(int64_t(E) * D), dim3(256), 0, st, input_edge, edge_out,
                             e.reverse, int64_t(E), D);
          launched();
        }
      }
    } else {
      float* node = md.f(int64_t(N) * Dn);
      if (N) {
        gather_rows(node, md.p("node_embedders.0.weight"), e.species, N, Dn, st);
        launched();
      }
      for (int L = 0; L < G; ++L) layer_fwd(L, node, input_edge, sv[L]);
      ro = readout_fwd(0, node, input_edge, net, false);
    }
    double* per_atom = per_atom_out ? per_atom_out : reinterpret_cast<double*>(md.f(2 * int64_t(N)));
    if (N) {
      hipLaunchKernelGGL(assemble_kernel, dim3(unsigned((N + 255) / 256)), dim3(256), 0, st, per_atom, net,
                         e.species, md.comp, md.h.energy_scale, N);
      launched();
    }
    if (energy) ok(pet_sum_by_structure(e.n_struct, 1, e.struct_off, per_atom, energy, 0, st));
    if (!grad) return;

    float* x4_adj = md.f(int64_t(E) * 4);
    float* cf_seq_adj = md.f(int64_t(N) * S);
    float* cutoff_adj = md.f(E);
    fill0(x4_adj, int64_t(E) * 4, st);
    fill0(cf_seq_adj, int64_t(N) * S, st);
    if (residual) {
      // each layer's tokens' adjoint from its read-out; ie_adj that of the next
      // layer's input_edge (src/residual.cpp:156-226)
      std::vector<float*> tadj(G);
      for (int L = 0; L < G; ++L) {
        tadj[L] = md.f(int64_t(T) * D);
        readout_bwd(L, rv[L].ro, tadj[L], tadj[L] + int64_t(N) * D, cutoff_adj, L > 0);
      }
      float* ie_adj = md.f(int64_t(E) * D);
      float* ie_next = md.f(int64_t(E) * D);
      for (int L = G - 1; L >= 0; --L) {
        float* efa = tadj[L] + int64_t(N) * D;
        if (L + 1 < G && E) {  // the message's reverse share: efa += ie_adj(rev) / 2
          hipLaunchKernelGGL(message_bwd_kernel, grid_for(int64_t(E) * D), dim3(256), 0, st, efa, ie_adj, e.reverse,
                             int64_t(E), D);
          launched();
        }
        float* tok_adj = residual_layer_bwd(L, rv[L], tadj[L], cf_seq_adj);
        // the message's own share: ie_next = ie_adj / 2 (0 past the last layer)
        if (E) {
          scale_pass(ie_next, ie_adj, L + 1 < G ? 0.5f : 0.0f, int64_t(E) * D, st);
        }
        compress_bwd(L, tok_adj + int64_t(N) * D, rv[L].cpre, x4_adj, ie_next);
        std::swap(ie_adj, ie_next);
      }
    } else {
      // backward (ff_pass, src/feedforward.cpp:396-410)
      float* node_adj = md.f(int64_t(N) * Dn);
      float* ie_adj = md.f(int64_t(E) * D);
      readout_bwd(0, ro, node_adj, ie_adj, cutoff_adj, false);
      for (int L = G - 1; L >= 0; --L) layer_bwd(L, sv[L], node_adj, ie_adj, x4_adj, cf_seq_adj);
    }

    // forces_and_virial (src/forces.cpp:345-386)
    double* grad_e = edge_grad_out ? edge_grad_out : reinterpret_cast<double*>(md.f(6 * int64_t(E)));
    ok(pet_edge_grad(N, E, e.off, e.center, x4_adj, 4, cutoff_adj, cf_seq_adj, S, e.vec, e.dist, e.pcut,
                     md.h.cutoff_width, md.h.cutoff_function, grad_e, st));
    double* vir_atom = reinterpret_cast<double*>(md.f(18 * int64_t(N)));
    ok(pet_fold_edge_gradients(N, N, e.off, e.reverse, e.vec, grad_e, md.h.energy_scale, forces, vir_atom, st));
    if (virial) ok(pet_sum_by_structure(e.n_struct, 9, e.struct_off, vir_atom, virial, 0, st));
  }
};

// Host-side load (src/model.cpp:180-289), in double.
struct Loader {
  const pet_model_hypers& h;
  std::unordered_map<std::string, const pet_model_tensor*> in;
  std::vector<std::pair<std::string, std::vector<float>>> out;
  std::vector<std::pair<int, int>> shapes;

  const pet_model_tensor& get(const std::string& n, int rows, int cols) const {
    auto it = in.find(n);
    if (it == in.end()) throw Error{PET_MODEL_EMISSING};
    const pet_model_tensor& t = *it->second;
    const int tc = t.cols ? t.cols : 1, want_c = cols ? cols : 1;
    if (t.rows != rows || tc != want_c || !t.data) throw Error{PET_MODEL_ESHAPE};
    return t;
  }
  void put(const std::string& n, int rows, int cols, const std::vector<double>& d) {
    std::vector<float> f(d.size());
    for (size_t i = 0; i < d.size(); ++i) f[i] = float(d[i]);
    out.emplace_back(n, std::move(f));
    shapes.emplace_back(rows, cols);
  }
  void copy(const std::string& n, int rows, int cols) {
    const pet_model_tensor& t = get(n, rows, cols);
    put(n, rows, cols ? cols : 1, std::vector<double>(t.data, t.data + size_t(rows) * (cols ? cols : 1)));
  }
  void linear(const std::string& p, int o, int i) { copy(p + ".weight", o, i), copy(p + ".bias", o, 0); }
  // [v | g] rows to (v_j, g_j) pairs (src/model.cpp:211-222)
  void swiglu_in(const std::string& p, int F2, int K) {
    const pet_model_tensor &W = get(p + ".weight", F2, K), &b = get(p + ".bias", F2, 0);
    const int F = F2 / 2;
    std::vector<double> w(size_t(F2) * K), bi(F2);
    for (int j = 0; j < F2; ++j) {
      const int src = j % 2 ? F + j / 2 : j / 2;
      std::memcpy(&w[size_t(j) * K], W.data + size_t(src) * K, sizeof(double) * K);
      bi[j] = b.data[src];
    }
    put(p + ".weight", F2, K, w);
    put(p + ".bias", F2, 1, bi);
  }
  // a linear's weight with the RMSNorm weight before it folded into its columns
  // (key@fold): norm(x) W^T = (1/rms(x)) x (W diag(w))^T
  void fold_norm(const std::string& lin, const std::string& nrm, int rows, int cols) {
    const pet_model_tensor &W = get(lin + ".weight", rows, cols), &w = get(nrm + ".weight", cols, 0);
    std::vector<double> f(size_t(rows) * cols);
    for (int r = 0; r < rows; ++r)
      for (int c = 0; c < cols; ++c) f[size_t(r) * cols + c] = W.data[size_t(r) * cols + c] * w.data[c];
    put(lin + "@fold.weight", rows, cols, f);
  }
  // compress.0 folded (src/model.cpp:236-262): its input is [edge_emb(x4) |
  // species table | input_edge], edge_emb linear in x4 = (v, |v|).
  void fold(int L) {
    const int D = h.d_pet, ns = h.n_species, K = (L == 0 ? 2 : 3) * D;
    const std::string g = "gnn_layers." + std::to_string(L), c0 = g + ".compress.0";
    const pet_model_tensor &W = get(c0 + ".weight", D, K), &b0 = get(c0 + ".bias", D, 0);
    const pet_model_tensor &We = get(g + ".edge_embedder.weight", D, 4), &be = get(g + ".edge_embedder.bias", D, 0);
    const pet_model_tensor& Tb = get(L == 0 ? "edge_embedder.weight" : g + ".neighbor_embedder.weight", ns, D);
    std::vector<double> wx(size_t(D) * 4, 0.0), b(b0.data, b0.data + D), tab(size_t(ns) * D, 0.0);
    for (int d = 0; d < D; ++d) {
      const double* wr = W.data + size_t(d) * K;
      for (int j = 0; j < D; ++j) {
        for (int c = 0; c < 4; ++c) wx[size_t(d) * 4 + c] += wr[j] * We.data[size_t(j) * 4 + c];
        b[d] += wr[j] * be.data[j];
        for (int s = 0; s < ns; ++s) tab[size_t(s) * D + d] += Tb.data[size_t(s) * D + j] * wr[D + j];
      }
    }
    put(c0 + "@x4", D, 4, wx);
    put(c0 + "@b", D, 1, b);
    put(c0 + "@tab", ns, D, tab);
    if (L == 0) return;
    std::vector<double> wi(size_t(D) * D);
    for (int d = 0; d < D; ++d)
      for (int j = 0; j < D; ++j) wi[size_t(d) * D + j] = W.data[size_t(d) * K + 2 * D + j];
    put(c0 + "@in", D, D, wi);
  }
};

}  // namespace

extern "C" {

int pet_model_create(const pet_model_hypers* hy, const pet_model_tensor* tensors, int n_tensors,
                     const double* composition, pet_model** out) {
  if (!hy || !out || (n_tensors > 0 && !tensors) || n_tensors < 0) return PET_ATTN_EINVAL;
  *out = nullptr;
  const pet_model_hypers& h = *hy;
  if (h.d_pet < 1 || h.d_node < 1 || h.d_head < 1 || h.num_heads < 1 || h.d_pet % h.num_heads ||
      h.num_gnn_layers < 1 || h.num_attention_layers < 1 || h.n_species < 1 || h.cutoff_function < 0 ||
      h.cutoff_function > 2 || !(h.cutoff_width > 0.0) || !(h.attention_temperature > 0.0) ||
      h.featurizer < 0 || h.featurizer > 1)
    return PET_ATTN_EINVAL;
  // the two families (src/model.cpp:326-336): feedforward with an expanded
  // central token (d_node != d_pet), residual without (d_node == d_pet)
  const bool residual = h.featurizer == 1;
  if (residual != (h.d_node == h.d_pet)) return PET_ATTN_EINVAL;
  // any head_dim the attention holds (1..128, the reference's kMaxHeadDim,
  // src/model.cpp:331-334): multiples of 16 on the LDS-staged kernels, the
  // rest on the streaming ones
  if (h.d_pet % h.num_heads) return PET_ATTN_EINVAL;
  const int hd = h.d_pet / h.num_heads;
  if (hd < 1 || hd > 128) return PET_ATTN_EHEADDIM;
  auto md = new pet_model();
  md->h = h, md->hd = hd;
  try {
    Loader ld{h, {}, {}, {}};
    for (int i = 0; i < n_tensors; ++i) {
      if (!tensors[i].name) throw Error{PET_ATTN_EINVAL};
      ld.in[tensors[i].name] = &tensors[i];
    }
    const int D = h.d_pet, Dn = h.d_node, Dh = h.d_head, ns = h.n_species;
    // the MLP widths from the checkpoint (ffn_pre_width, src/model.cpp:635)
    const std::string t0 = "gnn_layers.0.trans.layers.0";
    auto rows_of = [&](const std::string& n) {
      auto it = ld.in.find(n);
      if (it == ld.in.end()) throw Error{PET_MODEL_EMISSING};
      return it->second->rows;
    };
    md->ew = rows_of(t0 + ".mlp.w_in.weight"), md->cw = residual ? 0 : rows_of(t0 + ".center_mlp.w_in.weight");
    if (!residual && (md->ew % 2 || md->cw % 2)) throw Error{PET_MODEL_ESHAPE};
    for (int L = 0; L < h.num_gnn_layers; ++L) {
      const std::string g = "gnn_layers." + std::to_string(L), ls = std::to_string(L);
      ld.fold(L);
      ld.linear(g + ".compress.2", D, D);
      for (int a = 0; a < h.num_attention_layers; ++a) {
        const std::string tl = g + ".trans.layers." + std::to_string(a);
        ld.linear(tl + ".attention.input_linear", 3 * D, D);
        ld.linear(tl + ".attention.output_linear", D, D);
        ld.copy(tl + ".norm_attention.weight", D, 0);
        ld.copy(tl + ".norm_mlp.weight", D, 0);
        if (residual) {  // PostLN with LayerNorm, a SiLU MLP
          ld.copy(tl + ".norm_attention.bias", D, 0);
          ld.copy(tl + ".norm_mlp.bias", D, 0);
          ld.linear(tl + ".mlp.w_in", md->ew, D);
          ld.linear(tl + ".mlp.w_out", D, md->ew);
          continue;
        }
        ld.fold_norm(tl + ".attention.input_linear", tl + ".norm_attention", 3 * D, D);
        ld.swiglu_in(tl + ".mlp.w_in", md->ew, D);
        ld.linear(tl + ".mlp.w_out", D, md->ew / 2);
        ld.linear(tl + ".center_contraction", D, Dn);
        ld.linear(tl + ".center_expansion", Dn, D);
        ld.copy(tl + ".norm_center_features.weight", Dn, 0);
        ld.swiglu_in(tl + ".center_mlp.w_in", md->cw, Dn);
        ld.linear(tl + ".center_mlp.w_out", Dn, md->cw / 2);
      }
      if (residual) continue;
      ld.copy("combination_norms." + ls + ".weight", 2 * D, 0);
      ld.copy("combination_norms." + ls + ".bias", 2 * D, 0);
      ld.linear("combination_mlps." + ls + ".0", 2 * D, 2 * D);
      ld.linear("combination_mlps." + ls + ".2", D, 2 * D);
    }
    ld.copy("edge_embedder.weight", ns, D);
    // a read-out after every layer (residual) or once (feedforward)
    for (int i = 0; i < (residual ? h.num_gnn_layers : 1); ++i) {
      const std::string si = std::to_string(i);
      ld.copy("node_embedders." + si + ".weight", ns, Dn);
      ld.linear("node_heads.energy." + si + ".0", Dh, Dn);
      ld.linear("node_heads.energy." + si + ".2", Dh, Dh);
      ld.linear("edge_heads.energy." + si + ".0", Dh, D);
      ld.linear("edge_heads.energy." + si + ".2", Dh, Dh);
      ld.linear("node_last_layers.energy." + si + ".energy___0", 1, Dh);
      ld.linear("edge_last_layers.energy." + si + ".energy___0", 1, Dh);
    }

    // Every matrix also as its transpose ("name^T", [cols, rows]): a layer's
    // input adjoint out_adj W is then the same transposed-operand GEMM as the
    // forward (out_adj (W^T)^T), which rocBLAS runs 1.1-1.9x faster than the
    // non-transposed form at the models' shapes.
    for (size_t i = 0, n0 = ld.out.size(); i < n0; ++i) {
      const auto [rows, cols] = ld.shapes[i];
      if (cols <= 0) continue;
      const std::vector<float>& a = ld.out[i].second;
      std::vector<float> t(size_t(rows) * cols);
      for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) t[size_t(c) * rows + r] = a[size_t(r) * cols + c];
      ld.out.emplace_back(ld.out[i].first + "^T", std::move(t));
      ld.shapes.emplace_back(cols, rows);
    }
    size_t total = 0;
    std::vector<size_t> at;
    for (auto& [n, v] : ld.out) at.push_back(total), total += (sizeof(float) * v.size() + 255) & ~size_t(255);
    if (hipMalloc(&md->weights, total) != hipSuccess) throw Error{PET_MODEL_EMEMORY};
    std::vector<char> host(total, 0);
    for (size_t i = 0; i < ld.out.size(); ++i) {
      std::memcpy(host.data() + at[i], ld.out[i].second.data(), sizeof(float) * ld.out[i].second.size());
      md->m[ld.out[i].first] = {reinterpret_cast<float*>(static_cast<char*>(md->weights) + at[i]), ld.shapes[i].first,
                                ld.shapes[i].second};
    }
    if (hipMemcpy(md->weights, host.data(), total, hipMemcpyHostToDevice) != hipSuccess) throw Error{PET_ATTN_ELAUNCH};
    // split-row copies (at most 6 bytes an element) of the matrices whose K is a
    // multiple of 32, for the split-product dense layers
    size_t stotal = 0;
    std::vector<std::pair<const Mat*, size_t>> sat;
    for (auto& [n, mt] : md->m)
      if (mt.cols > 0 && mt.cols % 32 == 0)
        sat.push_back({&mt, stotal}), stotal += (size_t(6) * mt.rows * mt.cols + 255) & ~size_t(255);
    if (stotal) {
      if (hipMalloc(&md->wsplit, stotal) != hipSuccess) throw Error{PET_MODEL_EMEMORY};
      for (auto& [mt, o] : sat) {
        void* dst = static_cast<char*>(md->wsplit) + o;
        ok(pet_linear_split_weights(mt->p, mt->rows, mt->cols, mt->cols, dst, nullptr));
        md->split[mt->p] = dst;
      }
      if (hipDeviceSynchronize() != hipSuccess) throw Error{PET_ATTN_ELAUNCH};
    }
    // the matrices with K at most 128 as rows of three fp16 parts, for the short-K kernel
    std::vector<std::pair<const Mat*, size_t>> pat;
    size_t ptotal = 0;
    for (auto& [n, mt] : md->m)
      if (mt.cols > 0 && mt.cols <= 128 && mt.cols % 32 == 0)
        pat.push_back({&mt, ptotal}), ptotal += (size_t(6) * mt.rows * mt.cols + size_t(4) * mt.rows + 255) & ~size_t(255);
    if (ptotal) {
      if (hipMalloc(&md->wpair, ptotal) != hipSuccess) throw Error{PET_MODEL_EMEMORY};
      for (auto& [mt, o] : pat) {
        void* dst = static_cast<char*>(md->wpair) + o;
        ok(pet_gemm_pair_weights(mt->p, mt->rows, mt->cols, mt->cols, false, dst, nullptr));
        md->psplit[mt->p] = dst;
      }
      if (hipDeviceSynchronize() != hipSuccess) throw Error{PET_ATTN_ELAUNCH};
    }
    std::vector<double> comp(ns, 0.0);
    if (composition) comp.assign(composition, composition + ns);
    if (hipMalloc(&md->comp, sizeof(double) * ns) != hipSuccess) throw Error{PET_MODEL_EMEMORY};
    // the pairs scratch, where the device has room (else the products split
    // A as they stage it)
    if (md->wsplit && hipMalloc(&md->pairs, pet_model::kPairsBytes) != hipSuccess) {
      md->pairs = nullptr;
      (void) hipGetLastError();
    }
    if (hipMemcpy(md->comp, comp.data(), sizeof(double) * ns, hipMemcpyHostToDevice) != hipSuccess)
      throw Error{PET_ATTN_ELAUNCH};
  } catch (const Error& err) {
    delete md;
    return err.code;
  }
  *out = md;
  return PET_ATTN_OK;
}

void pet_model_destroy(pet_model* model) { delete model; }

namespace {
// The memory tier of an evaluation with forces (PetModel::recompute_tier,
// src/model.cpp:819-860, for the feedforward featurizer): option
// PET_OPT_MODEL_RECOMPUTE 1 or 2 forces "never" or "wide"; 0 takes "never"
// unless its estimate -- what the forward keeps plus the backward's largest
// temporaries, in floats: per block the token rows, qkv, merged, the edge MLP's
// pre-activation (E x ew) and the node/edge residual rows; per layer the
// combination's three 2D-wide edge arrays; the backward's E x ew and 1.5 T x
// 3D work -- passes 85% of what the device has free plus what the model's
// workspace already holds.
bool recompute_wide(const pet_model& md, const pet_model_edges& e) {
  const int opt = pet_attn_get_option(PET_OPT_MODEL_RECOMPUTE);
  if (opt) return opt == 2;
  const double N = e.n_atoms, E = e.n_edges, T = N + E, D = md.h.d_pet, Dn = md.h.d_node;
  const double G = md.h.num_gnn_layers, A = md.h.num_attention_layers;
  const double block = 5 * T * D + E * D + E * md.ew + N * (2 * Dn + md.cw) + T;
  const double never = 4.0 * (G * A * block + G * 5 * E * D + 1.5 * E * md.ew + 6 * T * D);
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return false;
  return never > 0.85 * (double(free_b) + double(md.ws.bytes()));
}
}  // namespace

int pet_model_last_tier(const pet_model* model) { return model ? model->tier : 0; }

size_t pet_model_workspace_bytes(const pet_model* model) { return model ? model->ws.bytes() : 0; }

size_t pet_model_pairs_scratch_bytes(const pet_model* model) {
  return model && model->pairs ? pet_model::kPairsBytes : 0;
}

int pet_model_compute(pet_model* md, const pet_model_edges* e, int forces, double* energy, double* per_atom,
                      double* forces_out, double* virial, double* edge_grad, void* stream) {
  if (!md || !e || e->n_atoms < 0 || e->n_edges < 0 || e->max_neighbors < 0 || e->n_struct < 0) return PET_ATTN_EINVAL;
  if (e->n_atoms == 0) return PET_ATTN_OK;
  md->gemm_mode = pet_attn_get_option(PET_OPT_MODEL_GEMM);
  md->blocks = pet_attn_get_option(PET_OPT_MODEL_PAIRS) == 1;
  if (!e->species || !e->off || (e->n_edges > 0 && (!e->center || !e->neigh_species || !e->reverse || !e->vec ||
                                                    !e->dist || !e->pcut || !e->cut)))
    return PET_ATTN_EINVAL;
  if (energy && (!e->struct_off || e->n_struct < 1)) return PET_ATTN_EINVAL;
  if (forces && (!forces_out || (virial && (!e->struct_off || e->n_struct < 1)))) return PET_ATTN_EINVAL;
  if (edge_grad && md->h.energy_scale != 1.0) return PET_ATTN_EINVAL;
  if (int64_t(e->n_atoms) + e->n_edges >= (int64_t(1) << 31) / std::max(std::max(3 * md->h.d_pet, md->ew), md->cw))
    return PET_ATTN_EINDEX;
  try {
    Pass p(*md, *e, reinterpret_cast<hipStream_t>(stream));
    p.wide = forces != 0 && md->h.featurizer == 0 && recompute_wide(*md, *e);
    md->tier = p.wide ? 2 : 1;
    p.run(forces != 0, energy, per_atom, forces_out, virial, edge_grad);
  } catch (const Error& err) {
    return err.code;
  }
  return PET_ATTN_OK;
}

}  // extern "C"
