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
  PET_ATTN_EHEADDIM = 2,    /* head_dim not one the kernels hold (a multiple of 16, <= 128) */
  PET_ATTN_ESLOTS = 3,      /* slots (S) above pet_attn_max_slots(head_dim) */
  PET_ATTN_EALIGN = 4,      /* a pointer or leading dimension not a multiple of 4 floats */
  PET_ATTN_ELAUNCH = 5,     /* a HIP launch or runtime call failed */
  PET_ATTN_EBLAS = 6,       /* the BLAS call of a linear failed */
  PET_ATTN_EWORKSPACE = 7,  /* the workspace is smaller than pet_attention_bwd_workspace() */
  PET_ATTN_EINDEX = 8       /* a row index or element offset that does not fit 2^31 */
};

/* The most tokens an atom may have (16 waves of 16 queries per workgroup). */
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

/* The most slots (S) both kernels hold for this head_dim on the current
 * device, their staged rows bounded by its LDS (at most PET_ATTN_MAX_SLOTS);
 * 0 for a head_dim they do not hold. Calls with a larger S return
 * PET_ATTN_ESLOTS. No counterpart in the reference, whose kernels stream
 * 16-token blocks through registers. */
PET_ATTN_API int pet_attn_max_slots(int head_dim);

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

#ifdef __cplusplus
}
#endif

#endif /* PET_ATTN_H */
