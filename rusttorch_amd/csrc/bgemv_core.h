// Device side of the batched decode GEMV (bgemv.hip): the tile-ordered MFMA
// GEMV unit, its epilogues and the LayerNorm statistics they carry. See
// bgemv.hip for the tile layout and the work split.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "argmax_key.h"
#include "bf16_split.h"

#include "bgemv.h"

namespace rtg {
namespace bgc {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

constexpr int DEPTH = 4;    // k-tiles in flight per wave of the streaming (ring) form
constexpr int SMAX = 8;     // most workgroups per panel group
constexpr int LNG_PER = 8;  // statistics groups per lane (ln_groups <= 128)


__device__ __forceinline__ float gelu_new_b(float x) {
  const float sqrt_2_pi = 0.7978845608028654f;  // gpt2.rs:837-847, the reference's association
  float inner = sqrt_2_pi * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <int WT>
struct Tile;
template <>
struct Tile<W_F32> {
  static constexpr int E = 4, TK = 16;
  typedef f4v Raw;
  __device__ __forceinline__ static float get(const Raw& w, int e) { return w[e]; }
};
template <>
struct Tile<W_BF16> {
  static constexpr int E = 8, TK = 32;
  typedef u4v Raw;
  // bf16_to_f32 = bits << 16 (nn/safetensors.rs:389-391)
  __device__ __forceinline__ static float get(const Raw& w, int e) {
    const unsigned u = w[e >> 1];
    return __uint_as_float((e & 1) ? (u & 0xffff0000u) : (u << 16));
  }
};

// The epilogue's operands for output (m, n) of one thread. The residual
// epilogue loads them before the k loop, so that the epilogue after it makes
// no global round trip before its stores (measured: 12.3 -> 11.7 us for
// 1600 x 6400 bf16 at M = 16); for the others, loading them early measured
// ~0.1 us slower, and they are loaded in the epilogue.
struct EpiIn {
  float bias, ln_s, g_next, resid;
};
__device__ __forceinline__ EpiIn load_epi(const BgemvArgs& a, int m, int n, bool lng) {
  EpiIn e{0.f, 0.f, 0.f, 0.f};
  if (n < a.N) {
    if (a.bias) e.bias = a.bias[n];
    if (lng) e.ln_s = a.ln_s[n];
    if (a.xg) e.g_next = a.g_next[n];
    if (!a.qkv.q && a.epi == EPI_BIAS_RESID && m < a.M) e.resid = a.C[(size_t)m * a.ldc + n];
  }
  return e;
}

// Applies the epilogue to v (row m, output n) and returns the value written;
// pos is the cache position of the new token (QKV epilogue only), tk the
// tile width of the input layout (c_tiled).
__device__ __forceinline__ float store_out(const BgemvArgs& a, int m, int n, float v, const EpiIn& e, int pos,
                                           int tk) {
  const float bv = e.bias;
  if (a.qkv.q) {
    // QKV epilogue: q to its buffer, the new token's k/v into the cache at
    // *pos_dev (LayerKVCache::append, gpt2.rs:500-514)
    const int d = a.qkv.d;
    if (n < d) {
      a.qkv.q[(size_t)m * a.qkv.ldq + n] = v + bv;
    } else {
      const int cc = n - (n < 2 * d ? d : 2 * d);
      const int hd = d / a.qkv.kv.n_head;
      const int h = cc / hd, dd = cc - h * hd;
      float* base = n < 2 * d ? a.qkv.kv.k : a.qkv.kv.v;
      base[(((size_t)m * a.qkv.kv.n_head + h) * a.qkv.kv.n_pos + pos) * hd + dd] = v + bv;
    }
    return v + bv;
  }
  float* cp = a.C + (a.c_tiled ? xt_index(m, n, a.M, tk) : (size_t)m * a.ldc + n);
  float y;
  if (a.epi == EPI_BIAS) y = v + bv;
  else if (a.epi == EPI_BIAS_GELU) y = gelu_new_b(v + bv);
  else if (a.epi == EPI_BIAS_RESID) y = e.resid + (v + bv);
  else y = v;
  *cp = y;
  return y;
}

// Sum over the 16 lanes of one DPP row (xor shuffles stay inside it).
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Residual epilogue statistics: this group's (mean, M2) per row over the
// columns it wrote, stored to stats_part[g][m] for the GEMV that reads x
// next. y[j] are the values thread tid (< 256) wrote (valid[j] false for
// columns past N or rows past M).
template <int NPW>
__device__ __forceinline__ void row_stats_partial(const BgemvArgs& a, int g, const float (&y)[NPW],
                                                  const bool (&valid)[NPW]) {
  const int tid = threadIdx.x, m = tid >> 4;
  float sum = 0.f, cnt = 0.f;
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    sum += valid[j] ? y[j] : 0.f;
    cnt += valid[j] ? 1.f : 0.f;
  }
  sum = row16_sum(sum);
  cnt = row16_sum(cnt);
  const float mean = cnt > 0.f ? sum / cnt : 0.f;
  float m2 = 0.f;
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const float t = y[j] - mean;
    m2 += valid[j] ? t * t : 0.f;
  }
  m2 = row16_sum(m2);
  if ((tid & 15) == 0 && m < a.M) {
    a.stats_part[((size_t)g * 16 + m) * 2] = mean;
    a.stats_part[((size_t)g * 16 + m) * 2 + 1] = m2;
  }
}

// LayerNorm statistics of input row m = tid / 16 from the producer's
// per-group partials (pv[i] = (mean, M2) of group sub + 16 i, sub = tid % 16):
// mean = sum_g n_g mean_g / K, var = sum_g (M2_g + n_g (mean_g - mean)^2) / K,
// each sum in a fixed order (per lane over its groups, then a fixed tree over
// the 16 lanes of the row).
__device__ __forceinline__ void row_stats_merge(const BgemvArgs& a, const float2 (&pv)[LNG_PER], float& mean,
                                                float& inv_std) {
  const int sub = threadIdx.x & 15;
  float s1 = 0.f;
#pragma unroll
  for (int i = 0; i < LNG_PER; ++i) {
    const int gg = sub + 16 * i;
    const float n = gg < a.ln_groups ? (float)min(a.ln_cols, a.K - gg * a.ln_cols) : 0.f;
    s1 += n * pv[i].x;
  }
  s1 = row16_sum(s1);
  mean = s1 / (float)a.K;
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < LNG_PER; ++i) {
    const int gg = sub + 16 * i;
    const float n = gg < a.ln_groups ? (float)min(a.ln_cols, a.K - gg * a.ln_cols) : 0.f;
    const float dm = pv[i].x - mean;
    s2 += n > 0.f ? pv[i].y + n * dm * dm : 0.f;
  }
  s2 = row16_sum(s2);
  inv_std = 1.0f / sqrtf(s2 / (float)a.K + a.eps);
}

// One work unit = panel group g, k split s, on the NW waves of this
// workgroup (wave w takes k-chunk s * NW + w). red: LDS [NW][NPW][256];
// last: one LDS word. Every thread of the workgroup calls it.
// DEPTH_ k-tiles of a wave are in flight at once: a ring refilled as tiles
// are consumed, or, with ONESHOT (the caller guarantees ktc <= DEPTH_), the
// whole chunk loaded at once and consumed without refills.
template <int WT, int NPW, bool LNG, int NW, int DEPTH_ = DEPTH, bool ONESHOT = false>
__device__ __forceinline__ void bgemv_unit(const BgemvArgs& a, int g, int s, float (*red)[NPW][256],
                                           unsigned* last) {
  typedef Tile<WT> TL;
  constexpr int E = TL::E, TK = TL::TK;
  typedef typename TL::Raw Raw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const bool ep = tid < 256;  // the epilogue threads: element tid of each panel
  const int NP = (a.N + 15) >> 4, KT = a.K / TK;
  const int chunk = s * NW + wave;
  const int t0 = min(KT, chunk * a.ktc), t1 = min(KT, t0 + a.ktc);
  const int nt = t1 - t0;
  const Raw* wp[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int p = min(g * NPW + j, NP - 1);
    wp[j] = reinterpret_cast<const Raw*>(a.Wt) + ((size_t)p * KT + t0) * 64 + lane;
  }
  // input layout xt_index: lane (r, q) loads chunk (h, q) of row r as 16
  // bytes at ((h * 4 + q) * M + r) * 4 within tile t (rows past M repeat the
  // last), so a group of 16 lanes reads M rows of one chunk contiguously
  const int xr = min(r, a.M - 1);
  const float* xb = a.X + (size_t)t0 * TK * a.M + (size_t)(q * a.M + xr) * 4;
  floatx4 acc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // DEPTH_ tiles in flight; past the end the last tile is re-read (never
  // consumed) so that the load sequence stays branch-free
  Raw w[DEPTH_][NPW];
  f4v x[DEPTH_][E / 4];
  auto issue = [&](int slot, int i) {
    const int ti = min(i, max(nt - 1, 0));
#pragma unroll
    for (int j = 0; j < NPW; ++j) w[slot][j] = __builtin_nontemporal_load(wp[j] + (size_t)ti * 64);
#pragma unroll
    for (int h = 0; h < E / 4; ++h)
      x[slot][h] = *reinterpret_cast<const f4v*>(xb + (size_t)ti * TK * a.M + h * 16 * a.M);
  };
  // one tile: acc += x . w over its TK inputs
  auto consume = [&](int d) {
    if constexpr (WT == W_BF16) {
      // bf16 weights: the tile is one v_mfma_f32_16x16x32_bf16 B operand;
      // x enters as three exact bf16 parts, so every product w * part is
      // exact in f32 and the MFMA accumulates in f32: the f32 GEMV up to
      // summation order (3 MFMAs per tile instead of 8 of 16x16x4 f32;
      // measured ~10% faster, with half the error against a float64 sum)
      float xs[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[e] = x[d][e >> 2][e & 3];
      u4v xh, xm, xl;
      split3(xs, xh, xm, xl);
#pragma unroll
      for (int j = 0; j < NPW; ++j) {
        const bf16x8 wb = as_bf16x8(w[d][j]);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xh), wb, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xm), wb, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xl), wb, acc[j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float xa = x[d][e >> 2][e & 3];
#pragma unroll
        for (int j = 0; j < NPW; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, TL::get(w[d][j], e), acc[j], 0, 0, 0);
      }
    }
  };
  // the input rows' LayerNorm statistics partials, loaded now and merged in
  // the epilogue (the kernel that wrote x left them)
  float2 lnp[LNG_PER];
  if (nt > 0) {
#pragma unroll
    for (int d = 0; d < DEPTH_; ++d) issue(d, d);
  }
  if constexpr (LNG) {
    const int mrow = min((tid & 255) >> 4, a.M - 1), sub = tid & 15;
#pragma unroll
    for (int i = 0; i < LNG_PER; ++i) {
      const int gg = min(sub + 16 * i, a.ln_groups - 1);
      lnp[i] = *reinterpret_cast<const float2*>(a.ln_part + ((size_t)gg * 16 + mrow) * 2);
    }
  }
  const int m = tid >> 4;
  const bool early = a.epi == EPI_BIAS_RESID && !a.qkv.q;
  EpiIn eo[NPW];
  if (ep && early) {
#pragma unroll
    for (int j = 0; j < NPW; ++j) eo[j] = load_epi(a, m, (g * NPW + j) * 16 + (tid & 15), LNG);
  }
  if (nt > 0) {
    if constexpr (ONESHOT) {
#pragma unroll
      for (int d = 0; d < DEPTH_; ++d)
        if (d < nt) consume(d);
    } else {
      for (int i0 = 0; i0 < nt; i0 += DEPTH_) {
#pragma unroll
        for (int d = 0; d < DEPTH_; ++d) {
          if (i0 + d < nt) consume(d);
          issue(d, i0 + d + DEPTH_);
        }
      }
    }
  }
  // partial D of this wave: element (m = 4q + i, n = r) at m*16 + n
#pragma unroll
  for (int j = 0; j < NPW; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][j][(4 * q + i) * 16 + r] = acc[j][i];
  __syncthreads();
  // this workgroup's sum over its waves, in wave order; thread tid owns element tid
  float v[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    float t = 0.f;
    if (ep) {
      t = red[0][j][tid];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) t += red[ww][j][tid];
    }
    v[j] = t;
  }
  if (a.S > 1) {
    // publish the workgroup partial (device-scope stores, complete before the
    // count), then the last of the S workgroups of this group sums them
    float* pg = a.part + ((size_t)g * a.S + s) * NPW * 256;
    if (ep) {
#pragma unroll
      for (int j = 0; j < NPW; ++j)
        __hip_atomic_store(pg + j * 256 + tid, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores have completed
    __syncthreads();
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(a.cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = old == (unsigned)(a.S - 1) ? 1u : 0u;
    }
    __syncthreads();
    const bool is_last = *last != 0u;
    __syncthreads();  // every thread has read *last before the next unit may write it
    if (!is_last) return;
    // all S partials in flight together (device-scope round trips), then
    // summed in split order
    const float* pb = a.part + (size_t)g * a.S * NPW * 256;
    if (ep) {
      float pv[SMAX][NPW];
#pragma unroll
      for (int ss = 0; ss < SMAX; ++ss)
#pragma unroll
        for (int j = 0; j < NPW; ++j)
          pv[ss][j] = ss < a.S ? __hip_atomic_load(const_cast<float*>(pb) + ((size_t)ss * NPW + j) * 256 + tid,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : 0.f;
#pragma unroll
      for (int j = 0; j < NPW; ++j) {
        float t = pv[0][j];
#pragma unroll
        for (int ss = 1; ss < SMAX; ++ss)
          if (ss < a.S) t += pv[ss][j];
        v[j] = t;
      }
    }
    if (tid == 0) __hip_atomic_store(a.cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!ep) {
    __syncthreads();  // the LDS partials are free again once the epilogue threads read them
    return;
  }
  float mean = 0.f, inv_std = 0.f, mc = 0.f;
  if constexpr (LNG) {
    row_stats_merge(a, lnp, mean, inv_std);
    // the input was centred on cen_in[m]: only the drift of the mean remains
    mc = mean - (a.cen_in && m < a.M ? a.cen_in[m] : 0.f);
    if (a.cen_out && g == 0 && (tid & 15) == 0 && m < a.M) a.cen_out[m] = mean;
  }
  const float xc = a.xg_cen && m < a.M ? a.xg_cen[m] : 0.f;
  if (!early) {
#pragma unroll
    for (int j = 0; j < NPW; ++j) eo[j] = load_epi(a, m, (g * NPW + j) * 16 + (tid & 15), LNG);
  }
  const int pos = a.qkv.q ? *a.qkv.pos_dev : 0;
  float y[NPW];
  bool valid[NPW];
  u64 best = 0ull;
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int n = (g * NPW + j) * 16 + (tid & 15);
    valid[j] = m < a.M && n < a.N;
    y[j] = 0.f;
    if (valid[j]) {
      float t = v[j];
      if constexpr (LNG) t = inv_std * (t - mc * eo[j].ln_s);
      y[j] = store_out(a, m, n, t, eo[j], pos, TK);
      if (a.xg) a.xg[xt_index(m, n, a.M, TK)] = (y[j] - xc) * eo[j].g_next;
      if (a.keys) {
        const u64 k = argmax_key(y[j], (uint32_t)n);
        best = k > best ? k : best;
      }
    }
  }
  if (a.stats_part) row_stats_partial<NPW>(a, g, y, valid);
  if (a.keys) {
    // greedy argmax of the LM head: the row's best key over this unit, then
    // one device-scope atomic max per row
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      const u64 other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if ((tid & 15) == 0 && m < a.M && best != 0ull)
      __hip_atomic_fetch_max(a.keys + m, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
}

}  // namespace bgc
}  // namespace rtg
