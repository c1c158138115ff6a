// Device side of decode attention for head dim 64 (one new token per
// sequence, multi_head_attention_cached, gpt2.rs:772-834) of the batched step
// (kernels.hip), plus cross-lane helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace rtg {

constexpr int AD_ITEM = 2 + 64;  // per-wave softmax state: m, l, o[64]

template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Pairwise combination with the lane 16 / 32 apart via gfx950's permlane
// swaps (VALU): the two swapped registers are the lane's value and its
// partner's, so their sum / max is the same in both lanes.
__device__ __forceinline__ float xor16_sum_k(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum_k(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max_k(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max_k(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float row16_sum_k(float v) {
  v += dpp_row<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_row<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_row<0x124>(v);  // row_ror:4
  v += dpp_row<0x128>(v);  // row_ror:8
  return v;
}

// exp(x) for the softmax, x <= 0: 2^(x log2 e) on the hardware exponent
// (v_exp_f32, about 1 ulp; exp(-inf) = 0) instead of the libm-accurate
// sequence (~15 instructions); the difference to the reference's f32 exp is
// far inside the logits tolerance.
__device__ __forceinline__ float fexp_a(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

constexpr int AF_RG = 4;  // row groups of 4 rows per window


// K/V rows of one window: row r0 + 4t + grp (clamped to len - 1), this lane's
// 4 dims at dq.
__device__ __forceinline__ void af_load(const float* Kh, const float* Vh, int r0, int len, int grp, int dq,
                                        float4 (&k4)[AF_RG], float4 (&v4)[AF_RG]) {
#pragma unroll
  for (int t = 0; t < AF_RG; ++t) {
    const int r = min(r0 + 4 * t + grp, len - 1);
    k4[t] = *reinterpret_cast<const float4*>(Kh + (size_t)r * 64 + dq);
    v4[t] = *reinterpret_cast<const float4*>(Vh + (size_t)r * 64 + dq);
  }
}

__device__ __forceinline__ void af_window(const float4 (&k4)[AF_RG], const float4 (&v4)[AF_RG], const float4& q4,
                                          int r0, int len, int grp, float& m, float& lsum, float4& o4) {
  float s[AF_RG];
  float mb = -INFINITY;
#pragma unroll
  for (int t = 0; t < AF_RG; ++t) {
    const float dot = row16_sum_k(q4.x * k4[t].x + q4.y * k4[t].y + q4.z * k4[t].z + q4.w * k4[t].w);
    s[t] = r0 + 4 * t + grp < len ? dot * 0.125f : -INFINITY;  // 1 / sqrt(64)
    mb = fmaxf(mb, s[t]);
  }
  mb = xor32_max_k(xor16_max_k(mb));
  const float mn = fmaxf(m, mb);
  const float corr = m == -INFINITY ? 0.f : fexp_a(m - mn);
  lsum *= corr;
  o4.x *= corr;
  o4.y *= corr;
  o4.z *= corr;
  o4.w *= corr;
#pragma unroll
  for (int t = 0; t < AF_RG; ++t) {
    const float p = s[t] == -INFINITY ? 0.f : fexp_a(s[t] - mn);
    lsum += p;
    o4.x += p * v4[t].x;
    o4.y += p * v4[t].y;
    o4.z += p * v4[t].z;
    o4.w += p * v4[t].w;
  }
  m = mn;
}

// Attention of (head h, sequence b) over positions [0, len) on the NWV waves
// of this workgroup: wave w takes the 16-row windows w, w + NWV, ... of the
// cache, each window's K/V rows loaded while the previous one is computed
// (two register sets), with an online softmax per wave (16 lanes per row, 4
// dims each, DPP row sums). The wave states (m, l, o) merge in LDS (wp,
// [NWV][AD_ITEM]) in wave order; out[b][h*64 + d] = o / l (row stride ldo),
// or with out_tk > 0 at xt_index(b, h*64 + d, B, out_tk). Every thread of the
// workgroup calls it.
template <int NWV>
__device__ __forceinline__ void attn_item(const float* __restrict__ q, int ldq, const float* __restrict__ kc,
                                          const float* __restrict__ vc, int H, int P, int len, int h, int b,
                                          float* __restrict__ out, int ldo, int out_tk, int B,
                                          float (*wp)[AD_ITEM]) {
  constexpr int WR = 4 * AF_RG;  // rows per window
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, grp = lane >> 4, dq = (lane & 15) * 4;
  const size_t head_off = ((size_t)b * H + h) * (size_t)P * 64;
  const float* Kh = kc + head_off;
  const float* Vh = vc + head_off;
  float m = -INFINITY, lsum = 0.f;
  float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  const int nwin = (len + WR - 1) / WR;
  if (wave < nwin) {
    const float4 q4 = *reinterpret_cast<const float4*>(q + (size_t)b * ldq + h * 64 + dq);
    float4 ka[AF_RG], va[AF_RG], kb[AF_RG], vb[AF_RG];
    af_load(Kh, Vh, wave * WR, len, grp, dq, ka, va);
    for (int w = wave; w < nwin; w += 2 * NWV) {
      const int wn = w + NWV;
      if (wn < nwin) af_load(Kh, Vh, wn * WR, len, grp, dq, kb, vb);
      af_window(ka, va, q4, w * WR, len, grp, m, lsum, o4);
      if (wn >= nwin) break;
      const int wn2 = wn + NWV;
      if (wn2 < nwin) af_load(Kh, Vh, wn2 * WR, len, grp, dq, ka, va);
      af_window(kb, vb, q4, wn * WR, len, grp, m, lsum, o4);
    }
    // sum over the 4 row groups
    lsum = xor32_sum_k(xor16_sum_k(lsum));
    o4.x = xor32_sum_k(xor16_sum_k(o4.x));
    o4.y = xor32_sum_k(xor16_sum_k(o4.y));
    o4.z = xor32_sum_k(xor16_sum_k(o4.z));
    o4.w = xor32_sum_k(xor16_sum_k(o4.w));
  }
  if (lane < 16) {
    wp[wave][2 + dq] = o4.x;
    wp[wave][3 + dq] = o4.y;
    wp[wave][4 + dq] = o4.z;
    wp[wave][5 + dq] = o4.w;
  }
  if (lane == 0) {
    wp[wave][0] = m;  // -inf (and l = 0) for a wave without rows
    wp[wave][1] = lsum;
  }
  __syncthreads();
  if (tid < 64) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) M = fmaxf(M, wp[w][0]);
    float Ls = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      const float mw = wp[w][0];
      const float f = mw == -INFINITY ? 0.f : fexp_a(mw - M);
      Ls += wp[w][1] * f;
      o += wp[w][2 + tid] * f;
    }
    const size_t oi = out_tk ? xt_index(b, h * 64 + tid, B, out_tk) : (size_t)b * ldo + h * 64 + tid;
    out[oi] = o / Ls;
  }
  __syncthreads();  // wp is free again
}

}  // namespace rtg
