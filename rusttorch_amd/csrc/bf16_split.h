// f32 values as exact sums of bf16 parts, for bf16 MFMAs that compute f32
// products exactly (the batched decode GEMV and the bf16-weight prefill GEMM).
#pragma once
#include <hip/hip_runtime.h>

namespace rtg {

typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// x as the exact sum hi + mid + lo of three bf16 values (each the top 16
// bits of an f32: hi = x truncated to bf16, mid = (x - hi) truncated, lo =
// x - hi - mid, whose at most 8 significant bits fit bf16 exactly), packed
// as the 8-element operand of a bf16 MFMA: dword i of a level holds elements
// 2i (low half) and 2i + 1.
__device__ __forceinline__ void split3(const float (&x)[8], u4v& hi, u4v& mid, u4v& lo) {
  unsigned bh[8], bm[8], bl[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const unsigned xb = __float_as_uint(x[e]);
    bh[e] = xb & 0xffff0000u;
    const float r1 = x[e] - __uint_as_float(bh[e]);
    bm[e] = __float_as_uint(r1) & 0xffff0000u;
    bl[e] = __float_as_uint(r1 - __uint_as_float(bm[e]));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    hi[i] = __builtin_amdgcn_perm(bh[2 * i + 1], bh[2 * i], 0x07060302u);
    mid[i] = __builtin_amdgcn_perm(bm[2 * i + 1], bm[2 * i], 0x07060302u);
    lo[i] = __builtin_amdgcn_perm(bl[2 * i + 1], bl[2 * i], 0x07060302u);
  }
}
__device__ __forceinline__ bf16x8 as_bf16x8(const u4v& v) { return __builtin_bit_cast(bf16x8, v); }

}  // namespace rtg
