// Split-fp32 products on gfx950's 16-bit matrix cores (bf16 parts, fp16 pairs), shared by the attention
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

// ---- fp32 products from fp16 pairs on the 16-bit matrix cores --------------
// A row of a matrix, scaled by a power of two s that puts its largest |x| in
// [2^14, 2^15), splits into two fp16 values per element, both rounded to
// nearest: hi = x s rounded to fp16 (its leading 11 bits) and lo = x s - hi
// (exact in fp32) rounded to fp16. hi + lo holds x to 2^-23 |x| (2^-25 of the
// row's largest where x s leaves fp16's normal range). A product a.b over k is
// then (a_hi b_hi + a_hi b_lo + a_lo b_hi) / (s_a s_b) with the three part
// products accumulated in fp32 by v_mfma_f32_16x16x32_f16 and the scales
// undone in the epilogue; the dropped a_lo b_lo is below 2^-22 |a||b| and,
// the lo parts of round-to-nearest splits having either sign, does not add
// up along k. (A truncated hi, whose lo always has x's sign, made the dropped
// terms share the product's sign: a bias along k of about 2^-21 of sum |a b|,
// which moved a d = 512 model's 648-atom energy 8.5e-6 from the float64
// oracle, against 1.5e-6 for the float32 oracle.) Three matrix instructions
// where the bf16 form takes six.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfma_h(const u4& a, const u4& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
// c += a.b with the fourth part product a_lo b_lo too: the error left is the
// rounding of the lo parts (2^-23 |a||b| at most, fp32's own order)
__device__ __forceinline__ f4 mfma4(const u4* a, const u4* b, f4 c) {
  c = mfma_h(a[1], b[1], c);
  c = mfma_h(a[1], b[0], c);
  c = mfma_h(a[0], b[1], c);
  return mfma_h(a[0], b[0], c);
}
// c += a.b from (hi, lo) parts, the small products first
__device__ __forceinline__ f4 mfma3(const u4* a, const u4* b, f4 c) {
  c = mfma_h(a[1], b[0], c);
  c = mfma_h(a[0], b[1], c);
  return mfma_h(a[0], b[0], c);
}
// two scaled values (exact products of a value and a power of two, or values
// as computed) as a register of hi parts and a register of lo parts, both to
// nearest
__device__ __forceinline__ void pair2(float x, float y, unsigned& hi, unsigned& lo) {
  const h2v h = {(_Float16)x, (_Float16)y};
  const h2v l = {(_Float16)(x - float(h[0])), (_Float16)(y - float(h[1]))};
  hi = __builtin_bit_cast(unsigned, h);
  lo = __builtin_bit_cast(unsigned, l);
}
// Two scaled values as three fp16 parts each, hi + mid + lo = the value
// exactly: hi its nearest fp16, mid the nearest fp16 of the rest (exact in
// fp32), lo what is left (at most 2 significant bits: exact in fp16 wherever
// the value is at least 2^-1; below that, within half an fp16 subnormal step).
// For a matrix used in many products: its representation error would be the
// same in every one of them, so none is left.
__device__ __forceinline__ void pair3(float x, float y, unsigned& hi, unsigned& mid, unsigned& lo) {
  const h2v h = {(_Float16)x, (_Float16)y};
  const float rx = x - float(h[0]), ry = y - float(h[1]);
  const h2v m = {(_Float16)rx, (_Float16)ry};
  const h2v l = {(_Float16)(rx - float(m[0])), (_Float16)(ry - float(m[1]))};
  hi = __builtin_bit_cast(unsigned, h);
  mid = __builtin_bit_cast(unsigned, m);
  lo = __builtin_bit_cast(unsigned, l);
}
// The row scale 2^(15 - e) for a largest |x| m = f 2^e (f in [0.5, 1)); 1 for
// a zero row (and for one holding a NaN, which then propagates).
__device__ __forceinline__ float pair_scale(float m) {
  if (!(m > 0.f) || m > 3.0e38f) return 1.f;
  const int e = __builtin_amdgcn_frexp_expf(m);
  return __builtin_amdgcn_ldexpf(1.f, min(15 - e, 126));
}

// The same pairs on the 16 x 16 x 16 instruction (k = 16: four fp16 values a
// lane, two registers), for products whose contraction is one 16-row block.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f4 mfma_h16(const u2& a, const u2& b, const f4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
}
// the same with a_lo b_lo too (as mfma4)
__device__ __forceinline__ f4 mfma4_16(const u2& ah, const u2& al, const u2& bh, const u2& bl, f4 c) {
  c = mfma_h16(al, bl, c);
  c = mfma_h16(al, bh, c);
  c = mfma_h16(ah, bl, c);
  return mfma_h16(ah, bh, c);
}
// c += a.b from (hi, lo) parts a = (ah, al), b = (bh, bl), the small products first
__device__ __forceinline__ f4 mfma3_16(const u2& ah, const u2& al, const u2& bh, const u2& bl, f4 c) {
  c = mfma_h16(al, bh, c);
  c = mfma_h16(ah, bl, c);
  return mfma_h16(ah, bh, c);
}

}  // namespace pet_split
