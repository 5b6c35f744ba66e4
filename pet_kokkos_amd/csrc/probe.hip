// The attention kernels' HBM access pattern alone, for measurement: the same
// grid, the same XCD-grouped item order and, per (atom, head) item, the same
// bytes read and written as attn_fwd_pair_kernel / attn_bwd_pair_kernel at
// head_dim 32 (a lane per (token slot, 8 dims): the forward reads its
// token's q, k and v slices and writes merged and the slot's (max, 1/sum);
// the backward reads q, k, v, dO and O and writes dq, dk, dv and the slot's
// cf share), with no arithmetic between but a sum that keeps every load
// live. Its time is the floor these kernels' memory traffic sets on this
// device, whatever their compute: what the fp16-pair kernels are measured
// against besides the 8 TB/s roofline. Writes only into the buffers given
// (the values are meaningless).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/pet_attn.h"
#include "attn_common.h"

namespace pet_attn {
namespace {

__global__ void __launch_bounds__(64 * 8) floor_fwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                           const int* __restrict__ off, int N, int S, int H,
                                                           float* __restrict__ merged, int64_t ldm, float* __restrict__ ml) {
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, 0, N);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4, i = 16 * w + c;
  if (w >= at.nb || i >= at.cnt) return;
  const int D = H * 32;
  const float* r = qkv + at.row(i) * ldq + at.h * 32 + 8 * g;
  float x[24];
  gmem_get<8>(r, x);
  gmem_get<8>(r + D, x + 8);
  gmem_get<8>(r + 2 * D, x + 16);
  float o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = x[t] + x[8 + t] + x[16 + t];
  float* m = merged + at.grow(i) * ldm + at.h * 32 + 8 * g;
  *reinterpret_cast<float4*>(m) = make_float4(o[0], o[1], o[2], o[3]);
  *reinterpret_cast<float4*>(m + 4) = make_float4(o[4], o[5], o[6], o[7]);
  if (g == 0) *reinterpret_cast<float2*>(ml + 2 * ((size_t(at.n) * H + at.h) * S + i)) = make_float2(o[0], o[1]);
}

__global__ void __launch_bounds__(64 * 8) floor_bwd_kernel(const float* __restrict__ qkv, int64_t ldq,
                                                           const int* __restrict__ off, int N, int S, int H,
                                                           const float* __restrict__ dmerged, int64_t ldg,
                                                           const float* __restrict__ merged, int64_t ldm,
                                                           float* __restrict__ qkv_adj, int64_t lda,
                                                           float* __restrict__ cfh) {
  const Atom at(off, xcd_item(blockIdx.x, gridDim.x), H, N, S, 0, N);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4, i = 16 * w + c;
  if (w >= at.nb || i >= at.cnt) return;
  const int D = H * 32;
  const size_t row = at.row(i);
  const float* r = qkv + row * ldq + at.h * 32 + 8 * g;
  float x[40];
  gmem_get<8>(r, x);
  gmem_get<8>(r + D, x + 8);
  gmem_get<8>(r + 2 * D, x + 16);
  gmem_get<8>(dmerged + row * ldg + at.h * 32 + 8 * g, x + 24);
  gmem_get<8>(merged + at.grow(i) * ldm + at.h * 32 + 8 * g, x + 32);
  float o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = x[t] + x[8 + t] + x[16 + t] + x[24 + t] + x[32 + t];
  float* a = qkv_adj + row * lda + at.h * 32 + 8 * g;
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    *reinterpret_cast<float4*>(a + m * D) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(a + m * D + 4) = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (g == 0) cfh[(size_t(at.n) * H + at.h) * S + i] = o[0];
}

}  // namespace
}  // namespace pet_attn

using namespace pet_attn;

extern "C" int pet_attn_access_floor(const pet_attn_shape* sh, int backward, const float* qkv, int64_t ldq,
                                     const int* off, const float* dmerged, int64_t ldg, float* merged, int64_t ldm,
                                     float* ml, float* qkv_adj, int64_t lda, float* cfh, void* stream) {
  if (!sh || sh->head_dim != 32 || sh->slots < 1 || sh->slots > 128 || sh->heads < 1 || sh->n_atoms < 0 || !off ||
      !qkv || !merged || (backward ? (!dmerged || !qkv_adj || !cfh) : !ml))
    return PET_ATTN_EINVAL;
  const int64_t items = int64_t(sh->n_atoms) * sh->heads;
  if (items == 0) return PET_ATTN_OK;
  if (items >= (int64_t(1) << 31)) return PET_ATTN_EINDEX;
  const int NW = (sh->slots + 15) / 16;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (backward)
    hipLaunchKernelGGL(floor_bwd_kernel, dim3(unsigned(items)), dim3(64 * NW), 0, st, qkv, ldq, off, sh->n_atoms,
                       sh->slots, sh->heads, dmerged, ldg, merged, ldm, qkv_adj, lda, cfh);
  else
    hipLaunchKernelGGL(floor_fwd_kernel, dim3(unsigned(items)), dim3(64 * NW), 0, st, qkv, ldq, off, sh->n_atoms,
                       sh->slots, sh->heads, merged, ldm, ml);
  return hipGetLastError() == hipSuccess ? PET_ATTN_OK : PET_ATTN_ELAUNCH;
}
