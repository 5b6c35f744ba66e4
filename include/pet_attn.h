/*
 * pet_attn.h -- the C ABI of the MI355X (gfx950) PET neighbourhood attention.
 *
 * PET's per-atom attention: atom n owns count(n) = 1 + (off[n+1] - off[n])
 * tokens, rows of one row-major token matrix of T = N + E rows: slot 0 is row
 * n (the atom's own token), slot s >= 1 is row N + off[n] + s - 1 (its s-th
 * kept edge). Per head h (columns h*hd .. h*hd+hd-1 of each of the Q, K, V
 * blocks of qkv = [Q | K | V], each D = H*hd wide), query i attends to key k
 * of the same atom with weight
 *     softmax_k( scale * q_i . k_k + log cf[n][k] ),
 * cf the smooth cutoff factor of slot k (1 for slot 0). A key with cf <= 0 is
 * left out; a query on an edge with cf <= 0 produces zeros. The backward
 * recomputes the weights from the saved per-query (max, 1/sum) and yields
 * dQ, dK, dV and each key's cutoff-factor adjoint.
 *
 * Conventions (those of the reference's attention()/attention_bwd(),
 * src/ops.hpp:121-148 of peterspackman/pet-kokkos):
 *   - every matrix is row-major fp32 with an explicit leading dimension (in
 *     elements); every pointer is device memory owned by the caller;
 *   - outputs that "accumulate" (cf_seq_adj) are added onto, everything else
 *     is overwritten; nothing here allocates device memory except the BLAS
 *     handle the op-level calls create once per device;
 *   - every call is enqueued on `stream` (a hipStream_t; NULL = the null
 *     stream) and returns without synchronising;
 *   - results are bit-identical from run to run: every sum has one owner and
 *     a fixed order, nothing is atomic.
 * Every function returns PET_ATTN_OK (0) or one of the error codes below.
 */
#ifndef PET_ATTN_H
#define PET_ATTN_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define PET_ATTN_API __attribute__((visibility("default")))
#else
#define PET_ATTN_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PET_ATTN_OK = 0,
  PET_ATTN_EINVAL = 1,      /* a null pointer, negative size or leading dimension too small */
  PET_ATTN_EHEADDIM = 2,    /* head_dim outside 1..128 (the reference's kMaxHeadDim, src/ops.hpp:19) */
  PET_ATTN_ESLOTS = 3,      /* slots (S) too large for a kernel that holds an atom in LDS (model-level callers) */
  PET_ATTN_EALIGN = 4,      /* a pointer or leading dimension not a multiple of 4 floats (head_dim a multiple of 4),
                               or a pointer not 4-byte aligned */
  PET_ATTN_ELAUNCH = 5,     /* a HIP launch or runtime call failed */
  PET_ATTN_EBLAS = 6,       /* the BLAS call of a linear failed */
  PET_ATTN_EWORKSPACE = 7,  /* the workspace is smaller than pet_attention_bwd_workspace() */
  PET_ATTN_EINDEX = 8,      /* a row index or element offset that does not fit 2^31 */
  PET_ATTN_ESCRATCH = 9     /* a size above pet_attn_bwd_noalloc's fixed scratch */
};

/* The most tokens an atom may have in the LDS-staged kernels (16 waves of 16
 * queries per workgroup); larger S runs on the streaming kernels. */
#define PET_ATTN_MAX_SLOTS 256

typedef struct pet_attn_shape {
  int n_atoms;   /* N: atoms whose tokens attend (the CSR off[] has N+1 entries) */
  int n_rows;    /* T = N + E: rows of qkv / merged / qkv_adj, E including dead capacity rows */
  int slots;     /* S: per-atom slots, >= every count(n); the width of cf_seq, ml and cfh */
  int heads;     /* H */
  int head_dim;  /* hd; D = H * hd */
  int dead;      /* nonzero: edge rows past N + off[N] exist and are zeroed (Tokens::dead) */
  float scale;   /* 1 / (sqrt(hd) * temperature), see pet_attn_scale() */
} pet_attn_shape;

/* scale = float(1 / (sqrt(double(hd)) * temperature)), the rounding of
 * src/attention.cpp:1525 (attention_impl). */
PET_ATTN_API float pet_attn_scale(int head_dim, double temperature);

PET_ATTN_API const char* pet_attn_strerror(int code);

/* The most slots (S) the LDS-staged kernels hold for this head_dim on the
 * current device (at most PET_ATTN_MAX_SLOTS); 0 for a head_dim they do not
 * hold (not a multiple of 16). Calls with a larger S, or such a head_dim, run
 * on the streaming kernels (keys or queries through LDS in 64-row tiles, any
 * S, any head_dim 1..128), as the reference computes any S on its flat path
 * and any head_dim on its generic one (src/attention.cpp:28-39, :195-203). */
PET_ATTN_API int pet_attn_max_slots(int head_dim);

/* ---- process-wide tuning options ----------------------------------------- */

/* Options that choose among equivalent kernels (all meet the same tolerance;
 * each choice is bit-repeatable). Defaults need none of them. They are
 * process-wide, read by each launch (an evaluation reads PET_OPT_MODEL_GEMM
 * once at its start), and not read from the environment. A HIP graph keeps the
 * kernels of the options in force when it was recorded. The reference's
 * counterpart is its process-global GEMM mode (include/pet/gemm.hpp:119-122). */
enum {
  PET_OPT_SPLIT = 1,       /* 1 (default): fp32 products split over the bf16 matrix cores where they pay; 0: fp32 MFMA only */
  PET_OPT_FWD_KERNEL = 2,  /* 0 (default): matrix-core forward, at head_dim 32 and 64 the fp16-pair one where it fits
                              (with PET_OPT_SPLIT 1); 1: the staged forward (split-bf16 scores where they pay);
                              3: the vector-ALU forward (head_dim <= 64), for comparison */
  PET_OPT_BWD_VLDS = 3,    /* 0 (default): automatic; 1: V staged in LDS; 2: V read from global memory (where it fits) */
  PET_OPT_BWD_NBUF = 4,    /* 0 (default): automatic; 1 or 2 backward tile buffers (where it fits) */
  PET_OPT_MODEL_GEMM = 5,  /* the model's dense layers: 6 (default) the split-product kernel for M*N*K >= 2^32, the
                              short-K kernel for the K <= 128 layers with a bias or activation in the epilogue and
                              N >= 64, rocBLAS for the rest; 4 as 6 without the short-K kernel; 5 this library's
                              kernels for every product (the short-K kernel for K <= 128, the split-product kernel
                              above), no result depending on M; 0 rocBLAS only; 1 / 2 the fp32 fused kernel for
                              every / <= 4096-row forward layer; 3 the split-product kernel wherever K is a multiple
                              of 32 */
  PET_OPT_ATTN_STREAM = 6, /* 0 (default): the LDS-staged kernels where they hold the shape; 1: the streaming kernels always */
  PET_OPT_BWD_KERNEL = 7,  /* 0 (default): at head_dim 32 and 64 the fp16-pair backward (every product on the 16-bit
                              matrix cores) where it fits, with PET_OPT_SPLIT 1; 1: the tile-exchange backward */
  PET_OPT_MODEL_RECOMPUTE = 8, /* the whole evaluation's memory tier (pet_model_compute): 0 (default) chosen from the
                              shapes and the device's free memory; 1 "never": every activation of the forward kept
                              for the backward; 2 "wide": the attention's qkv and the edge MLP's pre-activation not
                              kept but recomputed in the backward, the edge MLP run over chunks of edge rows (the
                              reference's Recompute::Wide, src/model.cpp:819-860) -- the same results */
  PET_OPT_MODEL_PAIRS = 9, /* the whole evaluation's MLPs: 1 (default) an activation, or its adjoint, that only the
                              next product reads passes to it as block pairs (pet_linear_fused_split_blocks /
                              pet_linear_fused_blocks) where both products take the pairs-by-pairs kernel; 0 as
                              fp32 and a split pass */
  PET_OPT_COUNT = 10
};

/* Sets an option; PET_ATTN_EINVAL for an unknown option or a value out of range. */
PET_ATTN_API int pet_attn_set_option(int option, int value);
/* The option's value, -1 for an unknown option. */
PET_ATTN_API int pet_attn_get_option(int option);

/* What pet_attn_fwd / pet_attn_bwd launch for a shape under the current
 * options, without launching: the streaming kernels, or the LDS-staged ones
 * with their split products and backward layout (used to price a roofline by
 * the instructions that run). No counterpart in the reference. */
typedef struct pet_attn_plan {
  int streaming;              /* 1: the streaming kernels (the fields below stay 0) */
  int waves;                  /* waves a workgroup (16 slots each) */
  int fwd_split_scores;       /* forward scores as split-fp32 products on the bf16 matrix cores */
  int fwd_valu;               /* the vector-ALU forward (option PET_OPT_FWD_KERNEL 3) */
  int fwd_lds_bytes, fwd_workgroups_per_cu;
  int bwd_split_dp;           /* backward dP as split-fp32 products on the bf16 matrix cores */
  int bwd_v_staged, bwd_tile_buffers;
  int bwd_lds_bytes, bwd_workgroups_per_cu;
  int bwd_pair;               /* the fp16-pair backward: every product as fp16 pairs on the 16-bit matrix cores */
  int fwd_pair;               /* the fp16-pair forward */
} pet_attn_plan;
PET_ATTN_API int pet_attn_describe(const pet_attn_shape* shape, pet_attn_plan* out);

/* ---- the core kernels -------------------------------------------------- */

/* Forward: merged[T, D] (ld ldm) = per-head attention of qkv[T, 3D] (ld ldq);
 * ml[N*H*S][2] = each query slot's (max, 1/sum), (-1e30, 0) for slots past an
 * atom's count and for cf <= 0 queries; ml may be NULL (nothing saved).
 * cf_seq is [N, S] with leading dimension ldc. Dead rows of merged are zeroed
 * when shape->dead.
 * Replaces the kernel half of attention_impl<HD> (reference
 * src/attention.cpp:1520-1558: Forward<HD>, mfma::forward<HD>, zero_dead). */
PET_ATTN_API int pet_attn_fwd(const pet_attn_shape* shape, const float* qkv, int64_t ldq, const int* off,
                 const float* cf_seq, int64_t ldc, float* merged, int64_t ldm, float* ml, void* stream);

/* Backward of the core: from dmerged [T, D] (ld ldg, the adjoint of merged),
 * the forward's merged (ld ldm) and ml, writes qkv_adj [T, 3D] (ld lda; dQ |
 * dK | dV, dead rows zeroed), cfh [N, H, S] (scratch: per atom, head and key
 * slot, the sum over queries of dS; the reference's cfh [N*S, H] transposed so
 * that one (atom, head) writes one contiguous row) and adds sum_h cfh / cf onto
 * cf_seq_adj [N, S] (ld ldca) where cf > 0.
 * Replaces the kernel half of attention_bwd_impl<HD> (reference
 * src/attention.cpp:1814-1907: Queries, Keys, mfma::backward, attn_bwd_cf,
 * zero_dead). */
PET_ATTN_API int pet_attn_bwd(const pet_attn_shape* shape, const float* qkv, int64_t ldq, const int* off,
                 const float* dmerged, int64_t ldg, const float* merged, int64_t ldm, const float* ml,
                 const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda, float* cfh,
                 float* cf_seq_adj, int64_t ldca, void* stream);

/* pet_attn_bwd for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * same kernels and the same results bit for bit, with no cfh argument -- its
 * N * H * S floats of scratch live in a fixed device array of
 * PET_ATTN_NOALLOC_MAX_SCRATCH bytes that the library holds on every GPU it
 * runs on until the process ends. Calls with N * heads * slots * 4 above that
 * size return PET_ATTN_ESCRATCH and launch nothing. The call allocates no
 * device memory. Its first call on a device (and the first launch of each
 * kernel shape) also looks the array's address up (hipGetSymbolAddress), may
 * raise a kernel's LDS limit (hipFuncSetAttribute) and records both in host
 * maps, which allocate host memory: make that first call outside graph
 * capture; later calls are capturable. All calls on one GPU share its array,
 * so calls that overlap on one GPU (on different streams, or from several
 * threads) race: order them on one stream. It has no counterpart in the
 * reference: it exists for the callers above, which cannot allocate. */
#define PET_ATTN_NOALLOC_MAX_SCRATCH (32u << 20)
PET_ATTN_API int pet_attn_bwd_noalloc(const pet_attn_shape* shape, const float* qkv, int64_t ldq, const int* off,
                                      const float* dmerged, int64_t ldg, const float* merged, int64_t ldm,
                                      const float* ml, const float* cf_seq, int64_t ldc, float* qkv_adj, int64_t lda,
                                      float* cf_seq_adj, int64_t ldca, void* stream);

/* For measurement: the HBM access pattern of the head_dim-32 fp16-pair kernels
 * alone -- their grid, item order and bytes (forward: q, k, v read, merged and
 * ml written; backward nonzero: q, k, v, dO, O read, qkv_adj and cfh
 * written) with no arithmetic between -- into the buffers given (values
 * meaningless). Its duration is the floor the kernels' traffic sets on the
 * device. Head_dim 32 and at most 128 slots only. No counterpart in the
 * reference: it calibrates the roofline. */
PET_ATTN_API int pet_attn_access_floor(const pet_attn_shape* shape, int backward, const float* qkv, int64_t ldq,
                                       const int* off, const float* dmerged, int64_t ldg, float* merged, int64_t ldm,
                                       float* ml, float* qkv_adj, int64_t lda, float* cfh, void* stream);

/* ---- runs of atoms: the kernels of attention_chunked / _bwd_chunked ------ */

/* pet_attn_fwd / pet_attn_bwd on qkv given as raw + transform: the attention
 * reads qkv[r][j] * row_scale[r] + bias[j] (row_scale [T] and bias [3D] each
 * may be NULL), so a QKV projection can leave its row scale and bias to the
 * attention: with qkv = tokens (W_in diag(norm_w))^T and row_scale = 1/rms(token),
 * this is the RMSNorm + input linear + attention of the reference's layer
 * without the normed tokens or a bias pass in memory. qkv_adj is the adjoint of
 * the transformed qkv. No counterpart in the reference (its attention reads a
 * finished qkv); the fused QKV projection's consumer (src/feedforward.cpp:107-123). */
PET_ATTN_API int pet_attn_fwd_xf(const pet_attn_shape* shape, const float* qkv, int64_t ldq, const float* row_scale,
                                 const float* bias, const int* off, const float* cf_seq, int64_t ldc, float* merged,
                                 int64_t ldm, float* ml, void* stream);
PET_ATTN_API int pet_attn_bwd_xf(const pet_attn_shape* shape, const float* qkv, int64_t ldq, const float* row_scale,
                                 const float* bias, const int* off, const float* dmerged, int64_t ldg,
                                 const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
                                 float* qkv_adj, int64_t lda, float* cfh, float* cf_seq_adj, int64_t ldca,
                                 void* stream);

/* The forward of atoms [n0, n1) only, whose token rows come as a chunk qkv
 * [Tc, 3D]: the run's own rows first (atom n at row n - n0), then its edges'
 * (edge k at row (n1 - n0) + k - e0), e0 = off[n0], Tc = (n1 - n0) +
 * off[n1] - e0 -- the chunk of the reference's attention_chunked (run_qkv,
 * src/attention.cpp:2055-2081). merged and ml are written at the whole's rows
 * (merged [T, D]) and slots; no dead rows are touched.
 * Replaces the per-run launch of mfma::forward in attention_chunked
 * (src/attention.cpp:2096-2117). */
PET_ATTN_API int pet_attn_fwd_run(const pet_attn_shape* shape, int n0, int n1, int e0, const float* qkv_chunk,
                                  int64_t ldq, const int* off, const float* cf_seq, int64_t ldc, float* merged,
                                  int64_t ldm, float* ml, void* stream);

/* The backward of atoms [n0, n1): qkv_chunk, dmerged_chunk [Tc, D] and
 * qkv_adj_chunk [Tc, 3D] in the run's chunk rows, merged (whole rows), ml and
 * cfh [N, H, S] at the whole's slots. No cf adjoint, no dead rows (see
 * pet_attn_cf_adjoint, pet_attn_zero_dead).
 * Replaces the per-run launch of mfma::backward in attention_bwd_chunked
 * (src/attention.cpp:2131-2171). */
PET_ATTN_API int pet_attn_bwd_run(const pet_attn_shape* shape, int n0, int n1, int e0, const float* qkv_chunk,
                                  int64_t ldq, const int* off, const float* dmerged_chunk, int64_t ldg,
                                  const float* merged, int64_t ldm, const float* ml, const float* cf_seq, int64_t ldc,
                                  float* qkv_adj_chunk, int64_t lda, float* cfh, void* stream);

/* cf_seq_adj[n][k] += (sum over heads h in order of cfh[n][h][k]) / cf_seq[n][k]
 * where cf_seq[n][k] > 0 -- the reference's attn_bwd_cf (src/attention.cpp:1829-1838). */
PET_ATTN_API int pet_attn_cf_adjoint(const pet_attn_shape* shape, const float* cfh, const float* cf_seq,
                                     int64_t ldc, float* cf_seq_adj, int64_t ldca, void* stream);

/* Rows N + off[N] .. T-1 of x [T, width] set to zero when shape->dead -- the
 * reference's zero_dead (src/attention.cpp:1510-1518). */
PET_ATTN_API int pet_attn_zero_dead(const pet_attn_shape* shape, float* x, int64_t ld, int width, const int* off,
                                    void* stream);

/* ---- the op level: attention() / attention_bwd() ----------------------- */

/* attention(): pet_attn_fwd into merged (ld D), then out[T, D] (ld ldo) =
 * merged . w_out^T + b_out (w_out [D, D] row-major, torch Linear layout;
 * b_out [D] or NULL). merged [T, D] and ml [N*H*S*2] are the saves the
 * backward reads (the reference keeps them in its Workspace under key+":merged"
 * and key+":ml"); ml may be NULL when nothing is saved.
 * Replaces pet::attention (reference src/ops.hpp:124-126,
 * src/attention.cpp:2189-2196). */
PET_ATTN_API int pet_attention(const pet_attn_shape* shape, float* out, int64_t ldo, const float* qkv, int64_t ldq,
                  const float* cf_seq, int64_t ldc, const float* w_out, const float* b_out,
                  const int* off, float* merged, float* ml, void* stream);

/* Bytes of device workspace pet_attention_bwd needs: dmerged [T, D],
 * qkv_adj [T, 3D] and cfh [N, H, S], each 256-byte aligned. */
PET_ATTN_API size_t pet_attention_bwd_workspace(const pet_attn_shape* shape);

/* attention_bwd(): dmerged = out_adj . w_out; the core backward; then
 * in_adj[T, d_in] (ld ldi) = qkv_adj . w_in + beta * in_adj (w_in [3D, d_in]
 * row-major), and cf_seq_adj += the cf adjoint. beta is 0 (overwrite) or any
 * other value (scale and accumulate), as linear_bwd's.
 * Replaces pet::attention_bwd (reference src/ops.hpp:129-132,
 * src/attention.cpp:2198-2206). */
PET_ATTN_API int pet_attention_bwd(const pet_attn_shape* shape, float* in_adj, int64_t ldi, int d_in, float* cf_seq_adj,
                      int64_t ldca, const float* out_adj, int64_t ldo, const float* qkv, int64_t ldq,
                      const float* cf_seq, int64_t ldc, const float* w_in, const float* w_out,
                      const int* off, const float* merged, const float* ml, float beta, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---- the op level over runs of atoms: attention_chunked() ---------------- */

/* Writes the qkv rows of tokens [r0, r1) of the whole token matrix into
 * qkv_rows (row 0 = token r0, leading dimension ld), enqueued on stream: the
 * reference's QkvRows (src/ops.hpp:136-139). */
typedef void (*pet_attn_make_qkv)(void* ctx, float* qkv_rows, int64_t ld, int r0, int r1, void* stream);

/* Bytes of device workspace attention_chunked and attention_bwd_chunked need
 * for runs of at most `chunk` tokens (atom_runs over off_host, the host copy of
 * off, N+1 entries): the run's qkv, dmerged and qkv_adj and cfh [N, H, S],
 * each 256-byte aligned. */
PET_ATTN_API size_t pet_attention_chunked_workspace(const pet_attn_shape* shape, const int* off_host, int chunk);

/* attention() over runs of consecutive atoms of about `chunk` tokens each
 * (at least one atom a run, the reference's atom_runs, src/attention.cpp:2060-2070),
 * so that qkv is only ever a run's rows, made by make_qkv: the same results
 * as pet_attention with the whole qkv. merged and ml are the saves.
 * Replaces pet::attention_chunked (src/ops.hpp:140-143, src/attention.cpp:2084-2129). */
PET_ATTN_API int pet_attention_chunked(const pet_attn_shape* shape, float* out, int64_t ldo, pet_attn_make_qkv make_qkv,
                                       void* ctx, const float* cf_seq, int64_t ldc, const float* w_out,
                                       const float* b_out, const int* off, const int* off_host, float* merged,
                                       float* ml, int chunk, void* workspace, size_t workspace_bytes, void* stream);

/* attention_bwd() over the same runs: per run dmerged = out_adj . w_out on its
 * rows, the core backward, in_adj rows = qkv_adj . w_in + beta * in_adj; then
 * the cf adjoint, and dead rows of in_adj scaled by beta (set to 0 when beta
 * is 0), as the whole's zeroed qkv adjoint gives them.
 * Replaces pet::attention_bwd_chunked (src/ops.hpp:144-146, src/attention.cpp:2131-2187). */
PET_ATTN_API int pet_attention_bwd_chunked(const pet_attn_shape* shape, float* in_adj, int64_t ldi, int d_in,
                                           float* cf_seq_adj, int64_t ldca, const float* out_adj, int64_t ldo,
                                           pet_attn_make_qkv make_qkv, void* ctx, const float* cf_seq, int64_t ldc,
                                           const float* w_in, const float* w_out, const int* off,
                                           const int* off_host, const float* merged, const float* ml, float beta,
                                           int chunk, void* workspace, size_t workspace_bytes, void* stream);

/* ---- the attention's input: cf_seq, the token norm and its callers -------- */

/* cf_seq[n][0] = 1, cf_seq[n][1 + m] = cut[off[n] + m] for m < off[n+1] - off[n],
 * 0 for the slots past the atom's count: the attention bias source, from each
 * kept edge's smooth cutoff factor in packed (CSR) order.
 * Replaces the device pet_cfseq pass (reference src/device_neighbors.cpp:318-323)
 * and its host twin (src/model.cpp:375-377). */
PET_ATTN_API int pet_attn_cf_seq(const pet_attn_shape* shape, const int* off, const float* cut, float* cf_seq,
                                 int64_t ldc, void* stream);

/* out[rows, width] = norm(in) row by row: RMSNorm, (x) / sqrt(mean(x^2) + eps)
 * * weight with eps = 2^-23, or LayerNorm when bias is not NULL, (x - mean) /
 * sqrt(var + 1e-5) * weight + bias; in fp32, the row's sums in a fixed order.
 * out may be in. Replaces norm_rows (reference src/ops.hpp:376-407). */
PET_ATTN_API int pet_norm_rows(int rows, int width, float* out, int64_t ldo, const float* in, int64_t ldi,
                               const float* weight, const float* bias, void* stream);

/* in_adj = beta * in_adj + the adjoint of norm(in) for out_adj, row by row:
 * inv (g w - [mean(g w), LayerNorm] - xhat mean(g w xhat)), xhat = (x - mu) inv.
 * beta 0 overwrites (in_adj is not read). ln nonzero: LayerNorm.
 * Replaces norm_rows_bwd (reference src/ops.hpp:409-436). */
PET_ATTN_API int pet_norm_rows_bwd(int rows, int width, float* in_adj, int64_t lda, float beta,
                                   const float* out_adj, int64_t ldg, const float* in, int64_t ldi,
                                   const float* weight, int ln, void* stream);

/* Bytes of device workspace pet_attention_layer / _layer_bwd need: the
 * normed tokens [T, D] and qkv [T, 3D], with pet_attention_bwd_workspace's,
 * each 256-byte aligned. */
PET_ATTN_API size_t pet_attention_layer_workspace(const pet_attn_shape* shape);

/* The attention of one PET layer from its tokens [T, D] (ld ldt): normed =
 * norm(tokens) (norm_w, norm_b: RMSNorm, or LayerNorm when norm_b is not NULL),
 * qkv = normed . w_in^T + b_in (w_in [3D, D]), then pet_attention into out
 * with the saves merged and ml.
 * Replaces the attention block of PetModel::ff_layer (reference
 * src/feedforward.cpp:96-123: norm_rows "norm_tok", linear, attention). */
PET_ATTN_API int pet_attention_layer(const pet_attn_shape* shape, float* out, int64_t ldo, const float* tokens,
                                     int64_t ldt, const float* norm_w, const float* norm_b, const float* w_in,
                                     const float* b_in, const float* cf_seq, int64_t ldc, const float* w_out,
                                     const float* b_out, const int* off, float* merged, float* ml,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* Its backward: normed and qkv rebuilt from tokens (as the reference's
 * rebuild()), pet_attention_bwd into the normed tokens' adjoint, then the
 * norm's backward into tokens_adj [T, D] (ld lda): rows < N set (beta 0) and
 * live edge rows N .. N + off[N] - 1 accumulated, as the reference's sink
 * (input_node_adj = g, edge_adj += g); dead rows untouched. cf_seq_adj
 * accumulates.
 * Replaces the attention block of PetModel::ff_layer_bwd (reference
 * src/feedforward.cpp:292-329: attention_bwd, norm_rows_bwd "norm_tok_bwd"). */
PET_ATTN_API int pet_attention_layer_bwd(const pet_attn_shape* shape, float* tokens_adj, int64_t lda,
                                         float* cf_seq_adj, int64_t ldca, const float* out_adj, int64_t ldo,
                                         const float* tokens, int64_t ldt, const float* norm_w, const float* norm_b,
                                         const float* w_in, const float* b_in, const float* cf_seq, int64_t ldc,
                                         const float* w_out, const int* off, const float* merged, const float* ml,
                                         void* workspace, size_t workspace_bytes, void* stream);

/* ---- the consumer of cf_seq_adj: the forces' edge term --------------------- */

/* Per packed edge k < off[n_centres] (of atom n = center[k], its m-th, m =
 * k - off[n]), in fp64:
 *   cutoff_total = cutoff_adj[k] + cf_seq_adj[n][1 + m],
 *   dist_adj     = x4_adj[k][3] + cutoff_total * dcf/dd(dist[k]; pcut[k], width),
 *   grad[k][c]   = x4_adj[k][c] + dist_adj * vec[k][c] / dist[k]   (0 at dist 0),
 * and grad = 0 for the dead rows k >= off[n_centres] up to n_edges. The
 * cutoff's derivative is in fp32 arithmetic as the reference evaluates it
 * (kind 0 bump, 1 cosine, 2 smooth). x4_adj [E, 4] (ld ldx) and cf_seq_adj
 * (ld ldca) are fp32; cutoff_adj [E] fp32 or NULL (zeros); vec [E, 3], dist,
 * pcut [E] and grad [E, 3] fp64.
 * Replaces the edge_grad pass of forces_and_virial (reference
 * src/forces.cpp:364-378, cutoff_ddist :21-42). */
PET_ATTN_API int pet_edge_grad(int n_centres, int n_edges, const int* off, const int* center, const float* x4_adj,
                               int64_t ldx, const float* cutoff_adj, const float* cf_seq_adj, int64_t ldca,
                               const double* vec, const double* dist, const double* pcut, double width, int kind,
                               double* grad, void* stream);

/* forces[i] = scale * sum over atom i's edges k (in order) of
 * (grad[k] - grad[reverse[k]]) (the reverse term where reverse[k] >= 0), and
 * virial_atom[i][3a + b] = scale * sum_k vec[k][a] grad[k][b], for atoms
 * i < n_atoms (those >= n_centres own no edges). fp64.
 * Replaces fold_edge_gradients' per-atom pass (reference src/forces.cpp:50-68). */
PET_ATTN_API int pet_fold_edge_gradients(int n_atoms, int n_centres, const int* off, const int* reverse,
                                         const double* vec, const double* grad, double scale, double* forces,
                                         double* virial_atom, void* stream);

/* out[b][t] (= or +=, accumulate nonzero) sum over atoms soff[b] .. soff[b+1]-1
 * of x[a][t], for n_struct structures and width columns, fp64, in a fixed order.
 * Replaces sum_by_structure (reference src/forces.cpp:287-302). */
PET_ATTN_API int pet_sum_by_structure(int n_struct, int width, const int* soff, const double* x, double* out,
                                      int accumulate, void* stream);

/* Each edge's geometry from positions, for a neighbour list kept between steps:
 * vec[e] = pos[neigh[e]] + shift[e] . cell - pos[center[e]] (cell [9] row-major,
 * lattice vectors as rows; shift [E, 3] ints, NULL for none), dist[e] = |vec[e]|
 * (1e30 for a coincident pair), pcut[e] = cutoff and cut[e] the smooth cutoff
 * factor of dist (kind 0 bump, 1 cosine, 2 smooth; transcendentals in fp32 as the
 * reference's CutT). positions [N, 3], cell, vec, dist, pcut fp64; cut fp32.
 * Pairs past the cutoff get factor 0 and weigh nothing in the model.
 * Replaces the per-step "nef_vectors" pass (reference src/device_geometry.cpp:
 * 335-345) and the cutoff factor of edge_geometry (src/device_neighbors.cpp:214-260,
 * include/pet/cutoff.hpp:17-40). */
PET_ATTN_API int pet_edge_geometry(int n_edges, const int* center, const int* neigh, const int* shift,
                                   const double* positions, const double* cell, double cutoff, double width, int kind,
                                   double* vec, double* dist, double* pcut, float* cut, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PET_ATTN_H */
