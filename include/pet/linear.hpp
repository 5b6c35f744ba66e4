// pet/linear.hpp -- the fused dense layers for a C++ caller: C = epilogue(A W^T)
// on gfx950's fp32 matrix cores (pet_linear_fused), or on its bf16 ones at
// fp32 accuracy from weights split once (pet::SplitWeights, with
// pet_linear_split_weights / pet_linear_fused_split).
//
// The reference's fused GEMMs by name (peterspackman/pet-kokkos src/ops.hpp:84-96,
// src/fused_gemm_hip.cpp:345-400): linear_fused (out = in W^T + b + beta out),
// silu_in_fused (out = silu(in W^T + b), pre kept) and swiglu_in_fused (pre =
// in W^T + b with W's rows interleaved value/gate, h = v sigmoid(g)). Row-major
// device pointers with their leading dimensions in place of Kokkos views; W is
// torch Linear's [N, K]. Each throws std::runtime_error on a bad shape or
// alignment where the reference returns false: there is no other path here.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../pet_model.h"

namespace pet {

inline void linear_check(int code, const char* what) {
  if (code) throw std::runtime_error(std::string("pet: ") + what + ": " + pet_attn_strerror(code));
}

// A weight matrix in either form: plain (W, ldw) or split.
struct DenseWeight {
  const float* w = nullptr;
  int64_t ldw = 0;
  const void* split = nullptr;  // set for the split form
  int rows = 0, cols = 0;       // N, K
};

// W [N, K] (ld ldw, K a multiple of 32) split once into device memory it owns.
class SplitWeights {
 public:
  SplitWeights(const float* W, int N, int K, int64_t ldw, hipStream_t stream = nullptr) : n_(N), k_(K) {
    if (hipMalloc(&p_, size_t(6) * N * K + 16) != hipSuccess) throw std::runtime_error("pet: SplitWeights: hipMalloc");
    const int e = pet_linear_split_weights(W, N, K, ldw, p_, stream);
    if (e) {
      (void) hipFree(p_);
      linear_check(e, "pet_linear_split_weights");
    }
  }
  SplitWeights(const SplitWeights&) = delete;
  SplitWeights& operator=(const SplitWeights&) = delete;
  ~SplitWeights() { (void) hipFree(p_); }
  DenseWeight weight() const { return {nullptr, 0, p_, n_, k_}; }

 private:
  void* p_ = nullptr;
  int n_, k_;
};

inline DenseWeight plain_weight(const float* W, int N, int K, int64_t ldw) { return {W, ldw, nullptr, N, K}; }

// An activation A [M, K] (ld lda, K a multiple of 32, at least 256) split once
// into fp16 pair rows in device memory it owns: the A operand of dense_pairs,
// which gives the bits of dense on A itself with W in the split form.
class PairRows {
 public:
  PairRows(const float* A, int M, int K, int64_t lda, hipStream_t stream = nullptr) : m_(M), k_(K) {
    if (hipMalloc(&p_, size_t(4) * M * K + size_t(4) * M + 16) != hipSuccess)
      throw std::runtime_error("pet: PairRows: hipMalloc");
    const int e = pet_linear_pair_rows(A, M, K, lda, p_, stream);
    if (e) {
      (void) hipFree(p_);
      linear_check(e, "pet_linear_pair_rows");
    }
  }
  PairRows(const PairRows&) = delete;
  PairRows& operator=(const PairRows&) = delete;
  ~PairRows() { (void) hipFree(p_); }
  const void* data() const { return p_; }
  int rows() const { return m_; }
  int cols() const { return k_; }

 private:
  void* p_ = nullptr;
  int m_, k_;
};

// dense() with A as pair rows; W must be split (SplitWeights::weight()).
inline void dense_pairs(const PairRows& A, const DenseWeight& W, float* C, int64_t ldc, const float* row_scale,
                        const float* bias, const float* cin, int64_t ldcin, float beta, float* pre, int64_t ldpre,
                        int act, hipStream_t stream) {
  if (!W.split || W.cols != A.cols()) throw std::runtime_error("pet: dense_pairs: W split with A's K is needed");
  linear_check(pet_linear_fused_pairs(A.rows(), W.rows, W.cols, A.data(), W.split, C, ldc, row_scale, bias, cin,
                                      ldcin, beta, pre, ldpre, act, stream),
               "pet_linear_fused_pairs");
}

// C = act(row_scale (A W^T) + bias + beta cin), pre = the value before act.
inline void dense(int M, const float* A, int64_t lda, const DenseWeight& W, float* C, int64_t ldc,
                  const float* row_scale, const float* bias, const float* cin, int64_t ldcin, float beta, float* pre,
                  int64_t ldpre, int act, hipStream_t stream) {
  if (W.split)
    linear_check(pet_linear_fused_split(M, W.rows, W.cols, A, lda, W.split, C, ldc, row_scale, bias, cin, ldcin, beta,
                                        pre, ldpre, act, stream),
                 "pet_linear_fused_split");
  else
    linear_check(pet_linear_fused(M, W.rows, W.cols, A, lda, W.w, W.ldw, C, ldc, row_scale, bias, cin, ldcin, beta,
                                  pre, ldpre, act, stream),
                 "pet_linear_fused");
}

// out [M, N] = in W^T + b + beta out
inline void linear_fused(float* out, int64_t ldo, const float* in, int64_t ldi, int M, const DenseWeight& W,
                         const float* b, float beta, hipStream_t stream = nullptr) {
  dense(M, in, ldi, W, out, ldo, nullptr, b, beta != 0.f ? out : nullptr, ldo, beta, nullptr, 0, 0, stream);
}
// out = silu(in W^T + b); pre (may be null) = in W^T + b
inline void silu_in_fused(float* out, float* pre, int64_t ld, const float* in, int64_t ldi, int M,
                          const DenseWeight& W, const float* b, hipStream_t stream = nullptr) {
  dense(M, in, ldi, W, out, ld, nullptr, b, nullptr, 0, 0.f, pre, ld, 1, stream);
}
// pre [M, N] = in W^T + b; h [M, N/2] (ld ldh; may be null) = v sigmoid(g)
inline void swiglu_in_fused(float* pre, int64_t ldp, float* h, int64_t ldh, const float* in, int64_t ldi, int M,
                            const DenseWeight& W, const float* b, hipStream_t stream = nullptr) {
  if (h)
    dense(M, in, ldi, W, h, ldh, nullptr, b, nullptr, 0, 0.f, pre, ldp, 2, stream);
  else
    dense(M, in, ldi, W, pre, ldp, nullptr, b, nullptr, 0, 0.f, nullptr, 0, 0, stream);
}

}  // namespace pet
