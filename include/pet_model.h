/* pet_model.h -- the whole PET energy / forces evaluation on gfx950 over a C ABI.
 *
 * The caller of the attention path: peterspackman/pet-kokkos's PetModel with
 * either featurizer it implements -- feedforward (PreLN, RMSNorm, SwiGLU,
 * d_node != d_pet: ff_pass / ff_layer / ff_layer_bwd, src/feedforward.cpp:34-411)
 * or residual (PostLN, LayerNorm, SiLU, d_node == d_pet, a readout after every
 * GNN layer: residual_pass / residual_layer, src/residual.cpp:13-251) -- with
 * its analytic backward, the readout and energy assembly
 * (src/model.cpp:656-780, src/ops.cpp:406-425) and forces_and_virial
 * (src/forces.cpp:345-386) for a fixed cutoff. Every kernel is this library's
 * (the attention, norms, activations, gathers, folds); the dense layers go to
 * rocBLAS fp32 with atomics off, so results repeat bit for bit.
 *
 * Weights come as the checkpoint stores them (include/pet/checkpoint.hpp,
 * src/model.cpp:180-289: torch Linear layout, a SwiGLU w_in as [value | gate]
 * rows, compress.0 unfolded); pet_model_create folds and interleaves them on
 * the host in double, as the reference's load_all does. All device buffers
 * of an evaluation come from a workspace the model owns and keeps between
 * calls (the reference's Workspace, include/pet/kokkos.hpp:65-84): after the
 * first call at a size, an evaluation allocates nothing.
 *
 * Return codes are pet_attn.h's PET_ATTN_* plus those below; pet_attn_strerror
 * names them all. One model serves one stream at a time: its workspace and
 * its pairs scratch are shared by every evaluation on it, so two
 * pet_model_compute calls on one model must not overlap (on two streams, or
 * from two threads); use one model per stream.
 */
#ifndef PET_MODEL_H
#define PET_MODEL_H

#include <stdint.h>

#include "pet_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PET_MODEL_EMISSING = 20, /* a tensor the architecture needs is not among those given */
  PET_MODEL_ESHAPE = 21,   /* a tensor's shape disagrees with the hyperparameters */
  PET_MODEL_EMEMORY = 22   /* a device allocation failed */
};

/* The hyperparameters evaluation needs (include/pet/config.hpp:30-70). */
typedef struct pet_model_hypers {
  int d_pet, d_node, d_head;
  int num_heads;             /* head_dim = d_pet / num_heads */
  int num_gnn_layers, num_attention_layers;
  int n_species;             /* rows of the embedding tables */
  int cutoff_function;       /* 0 bump, 1 cosine, 2 smooth (pet::CutoffFunction) */
  double cutoff_width;       /* the smooth cutoff's width */
  double attention_temperature;
  double energy_scale;       /* per-atom energy = energy_scale * net + composition[species] */
  int featurizer;            /* 0 feedforward, 1 residual (pet::FeaturizerType) */
} pet_model_hypers;

/* One checkpoint tensor, row-major float64 on the host: cols = 0 for a vector. */
typedef struct pet_model_tensor {
  const char* name;
  int rows, cols;
  const double* data;
} pet_model_tensor;

typedef struct pet_model pet_model;

/* Replaces PetModel::PetModel / load_all (src/model.cpp:61-112, :180-344):
 * uploads, folds compress.0 into its geometry matrix, bias, species table and
 * input_edge block, and (feedforward) interleaves each SwiGLU w_in to (v_j, g_j)
 * rows. The tensors a featurizer needs are those load_all reads for it.
 * composition [n_species] (may be null: zeros). Uses the current device. */
PET_ATTN_API int pet_model_create(const pet_model_hypers* hypers, const pet_model_tensor* tensors, int n_tensors,
                                  const double* composition, pet_model** out);
PET_ATTN_API void pet_model_destroy(pet_model* model);

/* A batch of structures with its kept edges, packed (the reference's
 * PackedEdges, include/pet/model.hpp:153-168, and DeviceEdgeData's species,
 * struct_id and max_neighbors, :60-112). All device pointers. */
typedef struct pet_model_edges {
  int n_atoms;         /* N; every atom is a centre */
  int n_edges;         /* E = off[N] */
  int max_neighbors;   /* M >= every atom's edge count; attention slots S = M + 1 */
  int n_struct;        /* B */
  const int* struct_off; /* [B + 1] atom offsets of the structures (contiguous atoms) */
  const int* species;    /* [N] species index */
  const int* off;        /* [N + 1] atom n's edges are off[n] .. off[n+1]-1 */
  const int* center;     /* [E] */
  const int* neigh_species; /* [E] the neighbour's species index */
  const int* reverse;    /* [E] the (j, i, -shift) edge, -1 if none */
  const double* vec;     /* [E, 3] r_j + shift - r_i */
  const double* dist;    /* [E] |vec| */
  const double* pcut;    /* [E] the pair cutoff (the cutoff factor's rc) */
  const float* cut;      /* [E] the smooth cutoff factor of dist */
} pet_model_edges;

/* One evaluation (PetModel::compute / energy_forces_batch, src/model.cpp:782-811,
 * :927-1010, with ff_pass src/feedforward.cpp:338-411). Outputs are device fp64:
 * energy [B], per_atom [N] (either may be null); with forces nonzero also
 * forces [N, 3], virial [B, 9] (row-major 3x3, W = sum v (x) dE/dv) and, unless
 * null, edge_grad [E, 3] (dE/dv per edge, scaled). */
PET_ATTN_API int pet_model_compute(pet_model* model, const pet_model_edges* edges, int forces, double* energy,
                                   double* per_atom, double* forces_out, double* virial, double* edge_grad,
                                   void* stream);

/* A dense layer on the fp32 matrix cores with its neighbours fused:
 *   v = (A W^T)[i][j] (A [M, K] ld lda, W [N, K] ld ldw, K a multiple of 16,
 *       A and W 16-byte aligned, lda and ldw multiples of 4),
 *   v *= row_scale[i], v += bias[j], v += beta * cin[i][j] (each when non-null),
 *   pre[i][j] = v (when non-null), then C[i][j] = v (act 0), silu(v) (act 1), or
 *   for act 2 (SwiGLU, W's rows interleaved value/gate) C[i][j/2] = v_j sigmoid(v_{j+1})
 *   for even j. cin may be C itself (a residual accumulated in place). A fixed
 *   summation order: results repeat bit for bit.
 * act 3 and 4 fuse an activation's backward instead: v = (A W^T)[i][j] is the
 *   adjoint of the activation's output, cin its saved pre-activation z (required;
 *   bias, when non-null, z's bias not yet added to it; row_scale, beta and pre
 *   unused, row_scale and pre must be null):
 *   act 3 (SiLU): C[i][j] = v silu'(z[i][j]);
 *   act 4 (SwiGLU, z [M, 2N] of interleaved (value u, gate g) pairs, C [M, 2N]):
 *   C[i][2j] = v sigmoid(g), C[i][2j+1] = v u sigmoid(g) (1 - sigmoid(g)),
 *   the adjoint of the pair (u, g) for h = u sigmoid(g).
 * Replaces the reference's fused GEMMs (src/fused_gemm_hip.cpp: linear_fused,
 * silu_in_fused, swiglu_in_fused; src/ops.hpp:84-96). */
PET_ATTN_API int pet_linear_fused(int M, int N, int K, const float* A, int64_t lda, const float* W, int64_t ldw,
                                  float* C, int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                  int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream);

/* The same dense layer with its products on the 16-bit matrix cores at fp32
 * accuracy; error at or below the fp32 instruction's. From K = 256 each row of
 * A and of W is scaled by a power of two and each element split into two fp16
 * parts (22 of its 24 significand bits), three part products accumulated in
 * fp32 and the scales undone in the epilogue; below K = 256 each fp32 operand
 * is split into three bf16 parts, the six part products whose order sum is at
 * most 2 accumulated in fp32. W is given split once by
 * pet_linear_split_weights: W [N, K] (ld ldw, K a multiple of 32) into out, at
 * most N * K * 6 bytes (N * K * 4 + N * 4 from K = 256), 16-byte aligned; the
 * form follows K, so a split copy always matches the product that reads it. pet_linear_fused_split then takes the split W in place of W and
 * ldw, K a multiple of 32, otherwise as pet_linear_fused; results repeat bit
 * for bit. No counterpart in the reference, which runs its dense layers in
 * fp32 (src/fused_gemm_hip.cpp); a faster form of pet_linear_fused. */
PET_ATTN_API int pet_linear_split_weights(const float* W, int N, int K, int64_t ldw, void* out, void* stream);
/* The split rows of B = W^T from W [K, N] (ld ldw >= N) without forming W^T:
 * what pet_linear_split_weights makes of W^T, for the input adjoint of a dense
 * layer (in_adj = out_adj W, i.e. B = W^T [K_in, N_out]). */
PET_ATTN_API int pet_linear_split_weights_transposed(const float* W, int N, int K, int64_t ldw, void* out,
                                                     void* stream);
PET_ATTN_API int pet_linear_fused_split(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit, float* C,
                                        int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                        int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream);
/* pet_linear_fused_split with a caller-owned device scratch (16-byte aligned):
 * where the product runs pairs by pairs (K >= 256, N >= 512) and the scratch
 * holds at least 128 rows of A as pairs (K * 4 + 4 bytes a row), A's rows are
 * split into it a chunk at a time (the largest multiple of 128 rows it
 * holds) and each chunk's product read from the pairs: the same bits as
 * without a scratch, A split once per row instead of once per column tile.
 * A smaller or null scratch takes the form without one. The model's large
 * products run this way from its own pairs scratch. */
PET_ATTN_API int pet_linear_fused_split_ws(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit,
                                           float* C, int64_t ldc, const float* row_scale, const float* bias,
                                           const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre,
                                           int act, void* scratch, size_t scratch_bytes, void* stream);

/* The dense layer for a short contraction, K at most 128 (a multiple of 32):
 * W [N, K] given by pet_linear_pair_weights as rows of three fp16 parts (W's
 * rows each scaled by a power of two and split into hi, mid and lo, which sum
 * to it exactly; N * K * 6 + N * 4 bytes, 16-byte aligned), A fp32 (lda a
 * multiple of 4, 16-byte aligned), epilogue as pet_linear_fused. The weights
 * of a wave's output columns stay in its registers; a workgroup splits each
 * 16-row block of A into fp16 pairs once for its four waves and runs five part
 * products on the 16-bit matrix cores (all but a_lo b_lo), so a row's results
 * depend on that row alone (not on M or the tiling) and repeat bit for bit. No counterpart in
 * the reference, which runs these layers in fp32 (src/fused_gemm_hip.cpp). */
PET_ATTN_API int pet_linear_pair_weights(const float* W, int N, int K, int64_t ldw, void* out, void* stream);
PET_ATTN_API int pet_linear_fused_smallk(int M, int N, int K, const float* A, int64_t lda, const void* Wpairs,
                                         float* C, int64_t ldc, const float* row_scale, const float* bias,
                                         const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre,
                                         int act, void* stream);

/* Activation rows as fp16 pairs, the A operand of pet_linear_fused_pairs: X [M, K]
 * (ld ldx, K a multiple of 32 and at least 256, rows 16-byte aligned) into out,
 * M * K * 4 + M * 4 bytes, 16-byte aligned (each row scaled by a power of two,
 * split into a high part exact in fp16 and the rest rounded to fp16, then the
 * rows' inverse scales). Split once, an activation feeds any number of products. */
PET_ATTN_API int pet_linear_pair_rows(const float* X, int M, int K, int64_t ldx, void* out, void* stream);
/* pet_norm_rows (RMSNorm, or LayerNorm with a bias) with its output as pair
 * rows: the bits pet_linear_pair_rows gives for pet_norm_rows' output, without
 * the fp32 round trip. width a multiple of 8 and at most 2048; out 16-byte
 * aligned, rows * width * 4 + rows * 4 bytes. */
PET_ATTN_API int pet_norm_rows_pairs(int rows, int width, void* out, const float* in, int64_t ldi,
                                     const float* weight, const float* bias, void* stream);
/* pet_linear_fused_split with A as pet_linear_pair_rows made it: the same bits,
 * with no arithmetic but the products in the K loop. No counterpart in the
 * reference (src/fused_gemm_hip.cpp runs its layers in fp32). */
PET_ATTN_API int pet_linear_fused_pairs(int M, int N, int K, const void* Apairs, const void* Wsplit, float* C,
                                        int64_t ldc, const float* row_scale, const float* bias, const float* cin,
                                        int64_t ldcin, float beta, float* pre, int64_t ldpre, int act, void* stream);

/* Block pairs: a product's output made directly as the fp16 pairs the next
 * product reads, with no fp32 round trip and no separate split pass.
 * pet_linear_fused_split_blocks is pet_linear_fused_split_ws (the pairs-by-pairs
 * path: K a multiple of 32 and at least 256, N >= 512 and a multiple of 128,
 * a scratch of at least 128 rows of A's pairs) with the epilogue's output
 * act(...) written into `out` instead of C: M rows of out_cols fp16 pairs
 * (out_cols = N / 2 for SwiGLU, 2 N for its backward, else N; a multiple of
 * 32), each row's 128-column tiles of the product scaled by their own power of
 * two (the largest |value| of the block at [2^14, 2^15)), then the blocks'
 * inverse scales [out_cols / kb][M]: M * out_cols * 4 + M * (out_cols / kb) * 4
 * bytes, 16-byte aligned. *kb receives the block width in output columns (64
 * for SwiGLU, 256 for its backward, 128 otherwise). Every epilogue operand
 * 16-byte aligned, leading dimensions multiples of 4.
 * pet_linear_fused_blocks is pet_linear_fused_pairs with A as such blocks (K =
 * out_cols, kb as returned, at most 32 blocks): each block's products summed
 * on their own, then into the total times the block's inverse scale. No
 * counterpart in the reference, whose fused layers (src/fused_gemm_hip.cpp:345-400)
 * write fp32. */
PET_ATTN_API int pet_linear_fused_split_blocks(int M, int N, int K, const float* A, int64_t lda, const void* Wsplit,
                                               void* out, const float* row_scale, const float* bias,
                                               const float* cin, int64_t ldcin, float beta, float* pre,
                                               int64_t ldpre, int act, void* scratch, size_t scratch_bytes, int* kb,
                                               void* stream);
PET_ATTN_API int pet_linear_fused_blocks(int M, int N, int K, const void* Ablocks, int kb, const void* Wsplit,
                                         float* C, int64_t ldc, const float* row_scale, const float* bias,
                                         const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre,
                                         int act, void* stream);

/* FLOPs (2 M N K per product) of the dense products this library's kernels
 * have launched in this process, by the instructions that run them:
 * flops[0] the fp32 fused kernel (fp32 matrix cores), [1] split-fp32 as bf16
 * parts (six bf16 products each), [2] fp16 pairs (three fp16 products), [3]
 * the short-K kernel (five fp16 products); products on rocBLAS are not
 * counted. reset != 0 zeroes the counts after reading them. A measurement aid
 * with no counterpart in the reference: the bench prices an evaluation's
 * products at the ceilings of the instructions that ran them. Counted at
 * launch, process-wide, from every thread. */
PET_ATTN_API int pet_gemm_flop_tally(double* flops, int reset);

/* Bytes of device workspace the model holds now (its high-water mark). */
PET_ATTN_API size_t pet_model_workspace_bytes(const pet_model* model);
/* Bytes of the model's pairs scratch (the large products' A operands as fp16
 * pairs, split once per activation): pet_model_create takes it where the
 * device has room; 0 when it has none, and then those products split A as
 * they stage it instead (the same bits, more work per product). */
PET_ATTN_API size_t pet_model_pairs_scratch_bytes(const pet_model* model);
/* The memory tier the model's last evaluation with forces ran (option
 * PET_OPT_MODEL_RECOMPUTE): 1 "never" (every activation kept), 2 "wide" (qkv
 * and the edge MLP's pre-activation remade in the backward, the edge MLP over
 * chunks of edge rows); 0 before any. The residual featurizer runs "never". */
PET_ATTN_API int pet_model_last_tier(const pet_model* model);

#ifdef __cplusplus
}
#endif

#endif /* PET_MODEL_H */
