// The op level of PET's attention: attention() and attention_bwd() as the
// reference's pet::attention / pet::attention_bwd run them
// (peterspackman/pet-kokkos src/attention.cpp:1520-1558, :1814-1907): the core
// kernels of attention.hip plus the output and input linears, whose GEMMs go to
// rocBLAS (fp32, atomics off so each product has one fixed summation order).
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <vector>

#include "../../include/pet_attn.h"

// gemm.hip: the split-product dense layer and its weight split
int pet_gemm_nt_split(int M, int N, int K, const float* A, int64_t lda, const void* Bs, float* C, int64_t ldc,
                      const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                      float* pre, int64_t ldpre, int act, hipStream_t st, void* scratch = nullptr,
                      size_t scratch_bytes = 0);
int pet_gemm_split_weights(const float* W, int N, int K, int64_t ldw, bool transposed, void* out, hipStream_t st);
int pet_gemm_nt_pp_blocks(int M, int N, int K, const void* Ap, int kb, const void* Bs, float* C, int64_t ldc,
                          const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta,
                          float* pre, int64_t ldpre, int act, hipStream_t st);
int pet_attn_bwd_xf_blocks(const pet_attn_shape* sh, const float* qkv, int64_t ldq, const float* rs, const float* b,
                           const int* off, const float* dmerged, int64_t ldg, const float* merged, int64_t ldm,
                           const float* ml, const float* cf_seq, int64_t ldc, void* qpairs, float* cfh,
                           float* cf_seq_adj, int64_t ldca, hipStream_t st);
int pet_gemm_nt_split_f32b(int M, int N, int K, const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                           int64_t ldc, const float* bias, const float* cin, int64_t ldcin, float beta, hipStream_t st);

namespace pet_attn {

// One rocBLAS handle per device, made on first use and kept for the process.
rocblas_handle blas_handle() {
  static std::mutex mu;
  static rocblas_handle handles[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!handles[dev]) {
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
    rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
    handles[dev] = h;
  }
  return handles[dev];
}

// out[M, Nout] (ld ldo, row-major) = in[M, K] W[Nout, K]^T + beta out.
int gemm_nt(float* out, int64_t ldo, const float* in, int64_t ldi, const float* W, int M, int Nout, int K, float beta,
            hipStream_t st) {
  rocblas_handle h = blas_handle();
  if (!h) return PET_ATTN_EBLAS;
  if (rocblas_set_stream(h, st) != rocblas_status_success) return PET_ATTN_EBLAS;
  const float one = 1.0f;
  // Column-major view: out^T [Nout, M] = W [Nout, K] (stored as W^T, lda K) . in^T [K, M].
  const rocblas_status s = rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, Nout, M, K, &one, W,
                                         K, in, rocblas_int(ldi), &beta, out, rocblas_int(ldo));
  return s == rocblas_status_success ? PET_ATTN_OK : PET_ATTN_EBLAS;
}
// in_adj[M, K] = out_adj[M, Nout] W[Nout, K] + beta in_adj.
int gemm_nn(float* in_adj, int64_t ldi, const float* out_adj, int64_t ldo, const float* W, int M, int Nout, int K,
            float beta, hipStream_t st) {
  rocblas_handle h = blas_handle();
  if (!h) return PET_ATTN_EBLAS;
  if (rocblas_set_stream(h, st) != rocblas_status_success) return PET_ATTN_EBLAS;
  const float one = 1.0f;
  // Column-major view: in_adj^T [K, M] = W^T [K, Nout] (W stored row-major, lda K) . out_adj^T [Nout, M].
  const rocblas_status s = rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_none, K, M, Nout, &one, W, K,
                                         out_adj, rocblas_int(ldo), &beta, in_adj, rocblas_int(ldi));
  return s == rocblas_status_success ? PET_ATTN_OK : PET_ATTN_EBLAS;
}

// The layer level's dense products on the split-product kernel (gemm.hip:
// fp32 accuracy on the bf16 matrix cores) where it was measured faster than
// rocBLAS -- products with M N K >= 2^32, K a multiple of 32 -- and the
// operands allow (A rows 16-byte aligned); split holds the weight's split
// rows (6 N K bytes) when the caller has room for them, else null.
// out[M, N] = A B^T (+ bias) + beta out, B [N, K] given as W = B (W_is_bt
// false, W [N, K] ld ldw) or W = B^T (true, W [K, N] ld ldw). Returns -1 when
// the split kernel does not take the product (the caller then runs rocBLAS).
int split_dense(float* out, int64_t ldo, const float* A, int64_t lda, const float* W, int64_t ldw, bool W_is_bt, int M,
                int N, int K, const float* bias, float beta, void* split, hipStream_t st) {
  if (!split || K % 32 || lda % 4 || (reinterpret_cast<uintptr_t>(A) & 15) || double(M) * N * K < 4294967296.0)
    return -1;
  if (int e = pet_gemm_split_weights(W, N, K, ldw, W_is_bt, split, st)) return e;
  return pet_gemm_nt_split(M, N, K, A, lda, split, out, ldo, nullptr, bias, beta != 0.f ? out : nullptr, ldo, beta,
                           nullptr, 0, 0, st);
}
// Bytes of split rows the layer level keeps for its four weights: W_in (folded)
// and W_in^T [3D x D each], W_out and W_out^T [D x D each].
inline size_t align256s(size_t n) { return (n + 255) & ~size_t(255); }
size_t layer_split_bytes(int D) {
  const size_t d = size_t(D);
  return 2 * align256s(6 * 3 * d * d) + 2 * align256s(6 * d * d);
}

// out[r][j] = b[j] (or 0 without a bias): the bias the GEMM then accumulates onto.
__global__ void fill_bias_kernel(float* __restrict__ out, int64_t ldo, const float* __restrict__ b, int M, int Nc) {
  const int64_t total = int64_t(M) * Nc;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = i / Nc;
    const int j = int(i - r * Nc);
    out[r * ldo + j] = b ? b[j] : 0.0f;
  }
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
// the backward's qkv_adj [T, 3D] in the workspace, with room for its block
// pairs' inverse scales (T 3H floats)
size_t qkv_adj_bytes(const pet_attn_shape& sh) {
  const size_t D = size_t(sh.heads) * sh.head_dim, T = size_t(sh.n_rows);
  return align256(sizeof(float) * T * (3 * D + 3 * size_t(sh.heads)));
}

// Rows N + off[N] .. T-1 of x [T, width]: 0 when beta is 0, else beta times
// themselves (what in_adj's dead rows get from a zeroed qkv adjoint).
__global__ void scale_dead_kernel(float* __restrict__ x, int64_t ld, int width, int N, int T,
                                  const int* __restrict__ off, float beta) {
  const int64_t first = int64_t(N) + off[N];
  const int64_t total = (int64_t(T) - N) * width;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = N + i / width;
    if (r >= first) {
      float* p = x + r * ld + (i % width);
      *p = beta == 0.0f ? 0.0f : beta * *p;
    }
  }
}

// Runs of consecutive atoms, each of at most about `chunk` tokens (at least
// one atom), with their first edges: the reference's atom_runs
// (src/attention.cpp:2060-2070).
struct Run {
  int n0, n1, e0, e1;
};
std::vector<Run> atom_runs(const int* off, int N, int chunk) {
  std::vector<Run> runs;
  for (int n0 = 0; n0 < N;) {
    int n1 = n0 + 1;
    while (n1 < N && (n1 + 1 - n0) + (off[n1 + 1] - off[n0]) <= chunk) ++n1;
    runs.push_back({n0, n1, off[n0], off[n1]});
    n0 = n1;
  }
  return runs;
}
int64_t max_run_rows(const std::vector<Run>& runs) {
  int64_t m = 0;
  for (const Run& r : runs) m = std::max<int64_t>(m, int64_t(r.n1 - r.n0) + (r.e1 - r.e0));
  return m;
}
struct ChunkWs {
  float *qkv, *dm, *qa, *cfh;
  size_t bytes;
};
ChunkWs chunk_ws(const pet_attn_shape& sh, int64_t rows, void* base) {
  const size_t D = size_t(sh.heads) * sh.head_dim, Tc = size_t(rows);
  const size_t a = align256(sizeof(float) * Tc * 3 * D), b = align256(sizeof(float) * Tc * D),
               c = align256(sizeof(float) * Tc * 3 * D),
               d = align256(sizeof(float) * size_t(sh.n_atoms) * sh.heads * sh.slots);
  char* p = static_cast<char*>(base);
  return {reinterpret_cast<float*>(p), reinterpret_cast<float*>(p + a), reinterpret_cast<float*>(p + a + b),
          reinterpret_cast<float*>(p + a + b + c), a + b + c + d};
}

}  // namespace pet_attn

using namespace pet_attn;

// rows.hip: the norm's backward with the reference's sink
int pet_rows_norm_bwd_sink(int rows, int width, float* in_adj, int64_t lda, const float* out_adj, int64_t ldg,
                           const float* in, int64_t ldi, const float* weight, int ln, int n_node, float beta_node,
                           float beta_edge, const int* live_off, hipStream_t st);
int pet_rows_rms_inv(int rows, int width, const float* in, int64_t ldi, float* inv, hipStream_t st);
int pet_rows_fold_cols(float* out, const float* w, const float* s, int rows, int cols, hipStream_t st);

namespace {

// qkv [T, 3D] = norm(tokens) . w_in^T + b_in, the normed tokens left in normed.
int layer_input(const pet_attn_shape* sh, float* normed, float* qkv, const float* tokens, int64_t ldt,
                const float* norm_w, const float* norm_b, const float* w_in, const float* b_in, hipStream_t st) {
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (int e = pet_norm_rows(T, D, normed, D, tokens, ldt, norm_w, norm_b, st)) return e;
  float beta = 0.0f;
  if (b_in) {
    const int64_t total = int64_t(T) * 3 * D;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(fill_bias_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, qkv,
                       int64_t(3) * D, b_in, T, 3 * D);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
    beta = 1.0f;
  }
  return gemm_nt(qkv, 3 * D, normed, D, w_in, T, 3 * D, D, beta, st);
}

// The fused QKV projection for an RMSNorm: inv = 1/rms(tokens), wf = w_in with
// the norm weight folded into its columns, qkv = tokens wf^T (no bias, no
// normed tokens); the attention applies inv and b_in as it loads qkv.
int layer_input_rms(const pet_attn_shape* sh, float* inv, float* wf, float* qkv, const float* tokens, int64_t ldt,
                    const float* norm_w, const float* w_in, hipStream_t st, void* split = nullptr) {
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (int e = pet_rows_rms_inv(T, D, tokens, ldt, inv, st)) return e;
  if (int e = pet_rows_fold_cols(wf, w_in, norm_w, 3 * D, D, st)) return e;
  const int se = split_dense(qkv, 3 * D, tokens, ldt, wf, D, false, T, 3 * D, D, nullptr, 0.0f, split, st);
  if (se >= 0) return se;
  return gemm_nt(qkv, 3 * D, tokens, ldt, wf, T, 3 * D, D, 0.0f, st);
}

// out = merged w_out^T + b_out
int output_linear(const pet_attn_shape* sh, float* out, int64_t ldo, const float* merged, const float* w_out,
                  const float* b_out, hipStream_t st, void* split = nullptr) {
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  const int se = split_dense(out, ldo, merged, D, w_out, D, false, T, D, D, b_out, 0.0f, split, st);
  if (se >= 0) return se;
  float beta = 0.0f;
  if (b_out) {
    const int64_t total = int64_t(T) * D;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(fill_bias_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, out, ldo,
                       b_out, T, D);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
    beta = 1.0f;
  }
  return gemm_nt(out, ldo, merged, D, w_out, T, D, D, beta, st);
}

// attention_bwd with qkv given raw + (rs, b) (pet_attn_bwd_xf), workspace as
// pet_attention_bwd's.
int attention_bwd_xf(const pet_attn_shape* sh, float* in_adj, int64_t ldi, int d_in, float* cf_seq_adj, int64_t ldca,
                     const float* out_adj, int64_t ldo, const float* qkv, int64_t ldq, const float* rs,
                     const float* b, const float* cf_seq, int64_t ldc, const float* w_in, const float* w_out,
                     const int* off, const float* merged, const float* ml, float beta, char* ws, hipStream_t st,
                     void* split_out_t = nullptr, void* split_in_t = nullptr) {
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  float* dmerged = reinterpret_cast<float*>(ws);
  float* qkv_adj = reinterpret_cast<float*>(ws + align256(sizeof(float) * size_t(T) * D));
  float* cfh = reinterpret_cast<float*>(ws + align256(sizeof(float) * size_t(T) * D) + qkv_adj_bytes(*sh));
  // dmerged = out_adj W_out: B = W_out^T; in_adj = qkv_adj W_in: B = W_in^T
  int se = split_dense(dmerged, D, out_adj, ldo, w_out, D, true, T, D, D, nullptr, 0.0f, split_out_t, st);
  if (se > 0) return se;
  if (se < 0)
    if (int e = gemm_nn(dmerged, D, out_adj, ldo, w_out, T, D, D, 0.0f, st)) return e;
  // the core's backward writing qkv_adj as block pairs (a scale per row, head
  // and q | k | v) and the input adjoint from them on the pairs-by-pairs
  // kernel, with no fp32 qkv_adj and no split pass of it, where the fp16-pair
  // backward takes the shape and the product is large enough for the split
  // kernel (C3 op level on MI355X: see pet_attention_bwd)
  if (split_in_t && 3 * D >= 256 && (3 * D) % 32 == 0 && double(T) * d_in * 3 * D >= 4294967296.0 && ldi % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(in_adj) & 15) == 0) {
    const int rc = pet_attn_bwd_xf_blocks(sh, qkv, ldq, rs, b, off, dmerged, D, merged, D, ml, cf_seq, ldc, qkv_adj,
                                          cfh, cf_seq_adj, ldca, st);
    if (rc == PET_ATTN_OK) {
      if (int e = pet_gemm_split_weights(w_in, d_in, 3 * D, d_in, true, split_in_t, st)) return e;
      return pet_gemm_nt_pp_blocks(T, d_in, 3 * D, qkv_adj, sh->head_dim, split_in_t, in_adj, ldi, nullptr, nullptr,
                                   beta != 0.f ? in_adj : nullptr, ldi, beta, nullptr, 0, 0, st);
    }
    if (rc != PET_ATTN_ESLOTS) return rc;
  }
  if (int e = pet_attn_bwd_xf(sh, qkv, ldq, rs, b, off, dmerged, D, merged, D, ml, cf_seq, ldc, qkv_adj, 3 * D, cfh,
                              cf_seq_adj, ldca, st))
    return e;
  se = split_dense(in_adj, ldi, qkv_adj, 3 * D, w_in, d_in, true, T, d_in, 3 * D, nullptr, beta, split_in_t, st);
  if (se >= 0) return se;
  return gemm_nn(in_adj, ldi, qkv_adj, 3 * D, w_in, T, 3 * D, d_in, beta, st);
}

}  // namespace

extern "C" {

int pet_attention(const pet_attn_shape* sh, float* out, int64_t ldo, const float* qkv, int64_t ldq,
                  const float* cf_seq, int64_t ldc, const float* w_out, const float* b_out, const int* off,
                  float* merged, float* ml, void* stream) {
  if (!sh || !out || !w_out || !merged) return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (ldo < D) return PET_ATTN_EINVAL;
  if (int e = pet_attn_fwd(sh, qkv, ldq, off, cf_seq, ldc, merged, D, ml, stream)) return e;
  if (T == 0) return PET_ATTN_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // the output linear on the split-product kernel with W_out split as it is
  // staged (no workspace here) and b_out in its epilogue, where it is large
  // enough to pay (M N K >= 2^32) and the operands allow; else rocBLAS
  if (double(T) * D * D >= 4294967296.0 && D % 32 == 0 && ldo % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(out) & 15) == 0 && (reinterpret_cast<uintptr_t>(w_out) & 15) == 0)
    return pet_gemm_nt_split_f32b(T, D, D, merged, D, w_out, D, out, ldo, b_out, nullptr, 0, 0.0f, st);
  float beta = 0.0f;
  if (b_out) {
    const int64_t total = int64_t(T) * D;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(fill_bias_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, out, ldo,
                       b_out, T, D);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
    beta = 1.0f;
  }
  return gemm_nt(out, ldo, merged, D, w_out, T, D, D, beta, st);
}

// The backward's workspace: dmerged [T, D], qkv_adj [T, 3D], cfh [N, H, S],
// then room for split rows of W_out^T (D x D) and W_in^T (d_in x 3D), sized
// for d_in up to D (the attention's own width; a wider d_in runs its product
// on rocBLAS).
size_t bwd_core_bytes(const pet_attn_shape* sh) {
  const size_t D = size_t(sh->heads) * sh->head_dim, T = size_t(sh->n_rows);
  return align256(sizeof(float) * T * D) + qkv_adj_bytes(*sh) +
         align256(sizeof(float) * size_t(sh->n_atoms) * sh->slots * sh->heads);
}
size_t bwd_split_bytes(const pet_attn_shape* sh) {
  const size_t D = size_t(sh->heads) * sh->head_dim;
  return align256(6 * D * D) + align256(6 * 3 * D * D);
}

size_t pet_attention_bwd_workspace(const pet_attn_shape* sh) {
  if (!sh) return 0;
  return bwd_core_bytes(sh) + bwd_split_bytes(sh);
}

int pet_attention_bwd(const pet_attn_shape* sh, float* in_adj, int64_t ldi, int d_in, float* cf_seq_adj,
                      int64_t ldca, const float* out_adj, int64_t ldo, const float* qkv, int64_t ldq,
                      const float* cf_seq, int64_t ldc, const float* w_in, const float* w_out, const int* off,
                      const float* merged, const float* ml, float beta, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (!sh || !in_adj || !out_adj || !w_in || !w_out || d_in < 1 || ldi < d_in) return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (ldo < D) return PET_ATTN_EINVAL;
  if (!workspace || workspace_bytes < pet_attention_bwd_workspace(sh)) return PET_ATTN_EWORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return PET_ATTN_EALIGN;
  if (T == 0) return PET_ATTN_OK;
  // both dense products on the split-product kernel where they are large
  // enough (M N K >= 2^32), from W_out^T and W_in^T split into the workspace
  // each call (a few microseconds): dmerged = out_adj W_out, in_adj = qkv_adj W_in
  char* ws = static_cast<char*>(workspace);
  char* split = ws + bwd_core_bytes(sh);
  void* split_in_t = d_in <= D ? split + align256(6 * size_t(D) * D) : nullptr;
  return attention_bwd_xf(sh, in_adj, ldi, d_in, cf_seq_adj, ldca, out_adj, ldo, qkv, ldq, nullptr, nullptr, cf_seq,
                          ldc, w_in, w_out, off, merged, ml, beta, ws, reinterpret_cast<hipStream_t>(stream), split,
                          split_in_t);
}

size_t pet_attention_chunked_workspace(const pet_attn_shape* sh, const int* off_host, int chunk) {
  if (!sh || !off_host || sh->n_atoms < 0) return 0;
  return chunk_ws(*sh, max_run_rows(atom_runs(off_host, sh->n_atoms, chunk)), nullptr).bytes;
}

int pet_attention_chunked(const pet_attn_shape* sh, float* out, int64_t ldo, pet_attn_make_qkv make_qkv, void* ctx,
                          const float* cf_seq, int64_t ldc, const float* w_out, const float* b_out, const int* off,
                          const int* off_host, float* merged, float* ml, int chunk, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (!sh || !out || !make_qkv || !w_out || !merged || !off_host) return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows, N = sh->n_atoms;
  if (ldo < D) return PET_ATTN_EINVAL;
  const std::vector<Run> runs = atom_runs(off_host, N, chunk);
  const ChunkWs ws = chunk_ws(*sh, max_run_rows(runs), workspace);
  if (!workspace || workspace_bytes < ws.bytes) return PET_ATTN_EWORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return PET_ATTN_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (const Run& r : runs) {
    const int Nc = r.n1 - r.n0;
    make_qkv(ctx, ws.qkv, 3 * D, r.n0, r.n1, stream);
    if (r.e1 > r.e0) make_qkv(ctx, ws.qkv + int64_t(Nc) * 3 * D, 3 * D, N + r.e0, N + r.e1, stream);
    if (int e = pet_attn_fwd_run(sh, r.n0, r.n1, r.e0, ws.qkv, 3 * D, off, cf_seq, ldc, merged, D, ml, stream))
      return e;
  }
  if (int e = pet_attn_zero_dead(sh, merged, D, D, off, stream)) return e;
  if (T == 0) return PET_ATTN_OK;
  float beta = 0.0f;
  if (b_out) {
    const int64_t total = int64_t(T) * D;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(fill_bias_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, out, ldo,
                       b_out, T, D);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
    beta = 1.0f;
  }
  return gemm_nt(out, ldo, merged, D, w_out, T, D, D, beta, st);
}

int pet_attention_bwd_chunked(const pet_attn_shape* sh, float* in_adj, int64_t ldi, int d_in, float* cf_seq_adj,
                              int64_t ldca, const float* out_adj, int64_t ldo, pet_attn_make_qkv make_qkv, void* ctx,
                              const float* cf_seq, int64_t ldc, const float* w_in, const float* w_out, const int* off,
                              const int* off_host, const float* merged, const float* ml, float beta, int chunk,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (!sh || !in_adj || !out_adj || !make_qkv || !w_in || !w_out || !off_host || d_in < 1 || ldi < d_in)
    return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows, N = sh->n_atoms;
  if (ldo < D) return PET_ATTN_EINVAL;
  const std::vector<Run> runs = atom_runs(off_host, N, chunk);
  const ChunkWs ws = chunk_ws(*sh, max_run_rows(runs), workspace);
  if (!workspace || workspace_bytes < ws.bytes) return PET_ATTN_EWORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return PET_ATTN_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  for (const Run& r : runs) {
    const int Nc = r.n1 - r.n0, Ec = r.e1 - r.e0;
    make_qkv(ctx, ws.qkv, 3 * D, r.n0, r.n1, stream);
    if (Ec > 0) make_qkv(ctx, ws.qkv + int64_t(Nc) * 3 * D, 3 * D, N + r.e0, N + r.e1, stream);
    if (int e = gemm_nn(ws.dm, D, out_adj + int64_t(r.n0) * ldo, ldo, w_out, Nc, D, D, 0.0f, st)) return e;
    if (Ec > 0)
      if (int e = gemm_nn(ws.dm + int64_t(Nc) * D, D, out_adj + (int64_t(N) + r.e0) * ldo, ldo, w_out, Ec, D, D, 0.0f,
                          st))
        return e;
    if (int e = pet_attn_bwd_run(sh, r.n0, r.n1, r.e0, ws.qkv, 3 * D, off, ws.dm, D, merged, D, ml, cf_seq, ldc,
                                 ws.qa, 3 * D, ws.cfh, stream))
      return e;
    if (int e = gemm_nn(in_adj + int64_t(r.n0) * ldi, ldi, ws.qa, 3 * D, w_in, Nc, 3 * D, d_in, beta, st)) return e;
    if (Ec > 0)
      if (int e = gemm_nn(in_adj + (int64_t(N) + r.e0) * ldi, ldi, ws.qa + int64_t(Nc) * 3 * D, 3 * D, w_in, Ec,
                          3 * D, d_in, beta, st))
        return e;
  }
  if (int e = pet_attn_cf_adjoint(sh, ws.cfh, cf_seq, ldc, cf_seq_adj, ldca, stream)) return e;
  if (sh->dead && T > N) {
    const int64_t total = (int64_t(T) - N) * d_in;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(scale_dead_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, in_adj,
                       ldi, d_in, N, T, off, beta);
    if (hipGetLastError() != hipSuccess) return PET_ATTN_ELAUNCH;
  }
  return PET_ATTN_OK;
}

// [T, D] normed tokens (or their adjoint) | [T, 3D] qkv | [T] 1/rms | [3D, D] folded w_in | the backward's
size_t pet_attention_layer_workspace(const pet_attn_shape* sh) {
  if (!sh) return 0;
  const size_t D = size_t(sh->heads) * sh->head_dim, T = size_t(sh->n_rows);
  return align256(sizeof(float) * T * D) + align256(sizeof(float) * T * 3 * D) + align256(sizeof(float) * T) +
         align256(sizeof(float) * 3 * D * D) + pet_attention_bwd_workspace(sh) + layer_split_bytes(int(D));
}

int pet_attention_layer(const pet_attn_shape* sh, float* out, int64_t ldo, const float* tokens, int64_t ldt,
                        const float* norm_w, const float* norm_b, const float* w_in, const float* b_in,
                        const float* cf_seq, int64_t ldc, const float* w_out, const float* b_out, const int* off,
                        float* merged, float* ml, void* workspace, size_t workspace_bytes, void* stream) {
  if (!sh || !tokens || !norm_w || !w_in) return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (ldt < D) return PET_ATTN_EINVAL;
  if (!workspace || workspace_bytes < pet_attention_layer_workspace(sh)) return PET_ATTN_EWORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return PET_ATTN_EALIGN;
  if (T == 0) return PET_ATTN_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const size_t a0 = align256(sizeof(float) * size_t(T) * D), a1 = align256(sizeof(float) * size_t(T) * 3 * D),
               a2 = align256(sizeof(float) * size_t(T));
  float* normed = reinterpret_cast<float*>(ws);
  float* qkv = reinterpret_cast<float*>(ws + a0);
  // the split rows of W_in (folded) and W_out, past the backward's workspace
  char* sp = ws + a0 + a1 + a2 + align256(sizeof(float) * 3 * size_t(D) * D) + pet_attention_bwd_workspace(sh);
  void* s_in = sp;
  void* s_out = sp + 2 * align256(6 * 3 * size_t(D) * D);
  if (!norm_b) {  // RMSNorm: the fused projection, norm and bias applied by the attention
    float *inv = reinterpret_cast<float*>(ws + a0 + a1), *wf = reinterpret_cast<float*>(ws + a0 + a1 + a2);
    if (int e = layer_input_rms(sh, inv, wf, qkv, tokens, ldt, norm_w, w_in, st, s_in)) return e;
    if (int e = pet_attn_fwd_xf(sh, qkv, 3 * D, inv, b_in, off, cf_seq, ldc, merged, D, ml, stream)) return e;
    return output_linear(sh, out, ldo, merged, w_out, b_out, st, s_out);
  }
  if (int e = layer_input(sh, normed, qkv, tokens, ldt, norm_w, norm_b, w_in, b_in, st)) return e;
  return pet_attention(sh, out, ldo, qkv, 3 * D, cf_seq, ldc, w_out, b_out, off, merged, ml, stream);
}

int pet_attention_layer_bwd(const pet_attn_shape* sh, float* tokens_adj, int64_t lda, float* cf_seq_adj, int64_t ldca,
                            const float* out_adj, int64_t ldo, const float* tokens, int64_t ldt, const float* norm_w,
                            const float* norm_b, const float* w_in, const float* b_in, const float* cf_seq,
                            int64_t ldc, const float* w_out, const int* off, const float* merged, const float* ml,
                            void* workspace, size_t workspace_bytes, void* stream) {
  if (!sh || !tokens_adj || !tokens || !norm_w || !w_in || !off) return PET_ATTN_EINVAL;
  const int D = sh->heads * sh->head_dim, T = sh->n_rows;
  if (ldt < D || lda < D) return PET_ATTN_EINVAL;
  if (!workspace || workspace_bytes < pet_attention_layer_workspace(sh)) return PET_ATTN_EWORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return PET_ATTN_EALIGN;
  if (T == 0) return PET_ATTN_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const size_t a0 = align256(sizeof(float) * size_t(T) * D), a1 = align256(sizeof(float) * size_t(T) * 3 * D),
               a2 = align256(sizeof(float) * size_t(T)), a3 = align256(sizeof(float) * 3 * size_t(D) * D);
  float* normed = reinterpret_cast<float*>(ws);
  float* qkv = reinterpret_cast<float*>(ws + a0);
  float* inv = nullptr;
  const float* bq = nullptr;
  // the split rows of W_in (folded), W_in^T and W_out^T, past the backward's workspace
  char* sp = ws + a0 + a1 + a2 + a3 + pet_attention_bwd_workspace(sh);
  void* s_in = sp;
  void* s_in_t = sp + align256(6 * 3 * size_t(D) * D);
  void* s_out_t = sp + 2 * align256(6 * 3 * size_t(D) * D) + align256(6 * size_t(D) * D);
  if (!norm_b) {  // RMSNorm: the fused projection (as the forward's)
    inv = reinterpret_cast<float*>(ws + a0 + a1);
    if (int e = layer_input_rms(sh, inv, reinterpret_cast<float*>(ws + a0 + a1 + a2), qkv, tokens, ldt, norm_w, w_in,
                                st, s_in))
      return e;
    bq = b_in;
  } else if (int e = layer_input(sh, normed, qkv, tokens, ldt, norm_w, norm_b, w_in, b_in, st)) {
    return e;
  }
  // the normed tokens' adjoint overwrites them: the backward reads only qkv
  if (int e = attention_bwd_xf(sh, normed, D, D, cf_seq_adj, ldca, out_adj, ldo, qkv, 3 * D, inv, bq, cf_seq, ldc,
                               w_in, w_out, off, merged, ml, 0.0f, ws + a0 + a1 + a2 + a3, st, s_out_t, s_in_t))
    return e;
  return pet_rows_norm_bwd_sink(T, D, tokens_adj, lda, normed, D, tokens, ldt, norm_w, norm_b != nullptr,
                                sh->n_atoms, 0.0f, 1.0f, off, st);
}

}  // extern "C"
