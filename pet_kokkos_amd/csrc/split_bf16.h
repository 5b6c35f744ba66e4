// Split-fp32 products on gfx950's bf16 matrix cores, shared by the attention
// kernels (attention.hip) and the dense layers (gemm.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace pet_split {

typedef float f4 __attribute__((ext_vector_type(4)));

// ---- fp32 products on the bf16 matrix cores ---------------------------------
// An fp32 x splits exactly into three bf16 values, x = x0 + x1 + x2 (each the
// truncated high half of an fp32: x0 takes x's leading 8 significand bits, x1
// the next 8 of the remainder, x2 what is left, at most 8 bits). A product
// a.b over k is then the sum of the six part products a_i.b_j with i + j <= 2,
// each exact in the fp32 accumulator; the three dropped are below 2^-24
// |a||b| (the "bf16x6" scheme, Henry, Tang & Heinecke, arXiv:1904.06376).
// gfx950's 16x16x32 bf16 MFMA issues in ~22 cycles against 32 for the 16x16x4
// fp32 one, so a k = 32 product takes 6 x 22 cycles instead of 8 x 32, at a
// measured error of 1.0e-7 of sum |a_k b_k| (fp32 MFMA: 1.9e-7). Operand
// layout as the fp32 instruction's, with k in 8-element groups: lane (c, g)
// holds row / column c, k = 8g .. 8g + 7, two bf16 a register.
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma_bf(const u4& a, const u4& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}
__device__ __forceinline__ void split3(float x, float& h0, float& h1, float& h2) {
  h0 = __uint_as_float(__float_as_uint(x) & 0xffff0000u);
  const float r1 = x - h0;  // exact
  h1 = __uint_as_float(__float_as_uint(r1) & 0xffff0000u);
  h2 = r1 - h1;  // exact, and at most 8 significant bits: its low half is zero
}
// Two bf16 in a register: x's high half low, y's high half high.
__device__ __forceinline__ unsigned pack_hi(float x, float y) {
  return __builtin_amdgcn_perm(__float_as_uint(y), __float_as_uint(x), 0x07060302u);
}
// Eight consecutive floats as three operand registers, part p in out[p].
__device__ __forceinline__ void split8(const float* x, u4* out) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float a0, a1, a2, b0, b1, b2;
    split3(x[2 * j], a0, a1, a2);
    split3(x[2 * j + 1], b0, b1, b2);
    out[0][j] = pack_hi(a0, b0), out[1][j] = pack_hi(a1, b1), out[2][j] = pack_hi(a2, b2);
  }
}
// c += a.b from split operands, the small products first.
__device__ __forceinline__ f4 mfma6(const u4* a, const u4* b, f4 c) {
  c = mfma_bf(a[1], b[1], c);
  c = mfma_bf(a[0], b[2], c);
  c = mfma_bf(a[2], b[0], c);
  c = mfma_bf(a[0], b[1], c);
  c = mfma_bf(a[1], b[0], c);
  return mfma_bf(a[0], b[0], c);
}

}  // namespace pet_split
