// Batched decode GEMV on fp32 MFMA for 2..16 sequences (the graph path of
// forward_cached with one new token per sequence, gpt2.rs:358-399 / 628-633):
// y[m][n] = epi(sum_k x[m][k] * W^T[n][k]) for m < M <= 16.
//
// The weights are read from a tile-ordered copy made once per model, so that
// every wave load is one contiguous KiB that lands in exactly the registers
// v_mfma_f32_16x16x4f32 takes as its B operand:
//   panel p    = output rows [16p, 16p + 16)
//   k-tile t   = inputs [t*TK, (t+1)*TK), TK = 16 (f32) or 32 (bf16)
//   tile (p,t) = 1 KiB; lane l = 16q + r holds the 16 bytes
//                W^T[16p + r][t*TK + q*E .. + E)  (E = 4 f32 / 8 bf16 values),
//                zeros past row N; tiles stored panel-major, [p][t].
// MFMA step e of a tile pairs k = t*TK + q*E + e for q = 0..3, so lane l's A
// operand is x[r][t*TK + q*E + e] and it accumulates D[4q + i][r], i < 4
// (batch row 4q + i, output row 16p + r).
//
// Work split: a wave owns NPW consecutive panels and one chunk of k-tiles; a
// workgroup's 4 waves take consecutive chunks of the same panels and sum them
// in LDS in wave order; with S > 1 workgroups per panel group the partials go
// to a workspace and the last workgroup to arrive (a per-group counter, reset
// by that workgroup) sums them in split order. Every sum has a fixed order, so
// results do not depend on timing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bgemv.h"

namespace rtg {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

constexpr int BG_NW = 4;     // waves per workgroup
constexpr int BG_DEPTH = 4;  // k-tiles in flight per wave
constexpr int BG_SMAX = 8;   // most workgroups per panel group
constexpr int BG_LNG_PER = 8;  // statistics groups per lane (ln_groups <= 128)
static_assert(BG_NW * 64 == 256, "the epilogues assume 256 threads");

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

__global__ void tile_weights_kernel(const void* __restrict__ src, int wtype, int N, int K, void* __restrict__ dst,
                                    long nchunks) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nchunks) return;
  const int E = wtype == W_F32 ? 4 : 8, TK = 4 * E, KT = K / TK;
  const int l = (int)(i & 63);
  const long pt = i >> 6;
  const int t = (int)(pt % KT);
  const long p = pt / KT;
  const long row = p * 16 + (l & 15);
  const int k = t * TK + (l >> 4) * E;
  u4v v = {0u, 0u, 0u, 0u};
  if (row < N) {
    const size_t off = ((size_t)row * K + k) * (wtype == W_F32 ? 4 : 2);
    v = *reinterpret_cast<const u4v*>(static_cast<const char*>(src) + off);
  }
  reinterpret_cast<u4v*>(dst)[i] = v;
}

// Applies the epilogue to v (row m, output n) and returns the value written.
__device__ __forceinline__ float store_out(const BgemvArgs& a, int m, int n, float v) {
  const float bv = a.bias ? a.bias[n] : 0.f;
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
      base[(((size_t)m * a.qkv.kv.n_head + h) * a.qkv.kv.n_pos + *a.qkv.pos_dev) * hd + dd] = v + bv;
    }
    return v + bv;
  }
  float* cp = a.C + (size_t)m * a.ldc + n;
  float y;
  if (a.epi == EPI_BIAS) y = v + bv;
  else if (a.epi == EPI_BIAS_GELU) y = gelu_new_b(v + bv);
  else if (a.epi == EPI_BIAS_RESID) y = *cp + (v + bv);
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
// columns it wrote, stored plainly to stats_part[g][m] (the next kernel reads
// them after the kernel boundary). y[j] are the values thread tid wrote
// (valid[j] false for columns past N or rows past M).
template <int NPW>
__device__ __forceinline__ void row_stats_partial(const BgemvArgs& a, const float (&y)[NPW], const bool (&valid)[NPW]) {
  const int tid = threadIdx.x, m = tid >> 4, g = blockIdx.x;
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
__device__ __forceinline__ void row_stats_merge(const BgemvArgs& a, const float2 (&pv)[BG_LNG_PER], float& mean,
                                                float& inv_std) {
  const int sub = threadIdx.x & 15;
  float s1 = 0.f;
#pragma unroll
  for (int i = 0; i < BG_LNG_PER; ++i) {
    const int gg = sub + 16 * i;
    const float n = gg < a.ln_groups ? (float)min(a.ln_cols, a.K - gg * a.ln_cols) : 0.f;
    s1 += n * pv[i].x;
  }
  s1 = row16_sum(s1);
  mean = s1 / (float)a.K;
  float s2 = 0.f;
#pragma unroll
  for (int i = 0; i < BG_LNG_PER; ++i) {
    const int gg = sub + 16 * i;
    const float n = gg < a.ln_groups ? (float)min(a.ln_cols, a.K - gg * a.ln_cols) : 0.f;
    const float dm = pv[i].x - mean;
    s2 += n > 0.f ? pv[i].y + n * dm * dm : 0.f;
  }
  s2 = row16_sum(s2);
  inv_std = 1.0f / sqrtf(s2 / (float)a.K + a.eps);
}

template <int WT, int NPW, bool LNG>
__global__ __launch_bounds__(64 * BG_NW) void bgemv_kernel(BgemvArgs a) {
  typedef Tile<WT> TL;
  constexpr int E = TL::E, TK = TL::TK;
  typedef typename TL::Raw Raw;
  __shared__ float red[BG_NW][NPW][256];
  __shared__ unsigned last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int g = blockIdx.x, s = blockIdx.y;
  const int NP = (a.N + 15) >> 4, KT = a.K / TK;
  const int chunk = s * BG_NW + wave;
  const int t0 = min(KT, chunk * a.ktc), t1 = min(KT, t0 + a.ktc);
  const int nt = t1 - t0;
  const Raw* wp[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int p = min(g * NPW + j, NP - 1);
    wp[j] = reinterpret_cast<const Raw*>(a.Wt) + ((size_t)p * KT + t0) * 64 + lane;
  }
  const float* xrow = a.X + (size_t)min(r, a.M - 1) * a.ldx + t0 * TK + q * E;
  const float* grow = a.ln_g + t0 * TK + q * E;  // LayerNorm gain at the same k (LNG)
  floatx4 acc[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // ring of BG_DEPTH tiles in flight; past the end the last tile is re-read
  // (never consumed) so that the load sequence stays branch-free
  Raw w[BG_DEPTH][NPW];
  f4v x[BG_DEPTH][E / 4];
  f4v gv[LNG ? BG_DEPTH : 1][E / 4];
  auto issue = [&](int slot, int i) {
    const int ti = min(i, max(nt - 1, 0));
#pragma unroll
    for (int j = 0; j < NPW; ++j) w[slot][j] = __builtin_nontemporal_load(wp[j] + (size_t)ti * 64);
#pragma unroll
    for (int h = 0; h < E / 4; ++h) {
      x[slot][h] = *reinterpret_cast<const f4v*>(xrow + ti * TK + 4 * h);
      if constexpr (LNG) gv[slot][h] = *reinterpret_cast<const f4v*>(grow + ti * TK + 4 * h);
    }
  };
  // the input rows' LayerNorm statistics partials, loaded now and merged in
  // the epilogue (they were written by the previous kernel)
  float2 lnp[BG_LNG_PER];
  if (nt > 0) {
#pragma unroll
    for (int d = 0; d < BG_DEPTH; ++d) issue(d, d);
  }
  if constexpr (LNG) {
    const int mrow = min(tid >> 4, a.M - 1), sub = tid & 15;
#pragma unroll
    for (int i = 0; i < BG_LNG_PER; ++i) {
      const int gg = min(sub + 16 * i, a.ln_groups - 1);
      lnp[i] = *reinterpret_cast<const float2*>(a.ln_part + ((size_t)gg * 16 + mrow) * 2);
    }
  }
  if (nt > 0) {
    for (int i0 = 0; i0 < nt; i0 += BG_DEPTH) {
#pragma unroll
      for (int d = 0; d < BG_DEPTH; ++d) {
        if (i0 + d < nt) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            float xa = x[d][e >> 2][e & 3];
            if constexpr (LNG) xa *= gv[d][e >> 2][e & 3];
#pragma unroll
            for (int j = 0; j < NPW; ++j)
              acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, TL::get(w[d][j], e), acc[j], 0, 0, 0);
          }
        }
        issue(d, i0 + d + BG_DEPTH);
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
    float t = red[0][j][tid];
#pragma unroll
    for (int ww = 1; ww < BG_NW; ++ww) t += red[ww][j][tid];
    v[j] = t;
  }
  if (a.S > 1) {
    // publish the workgroup partial (device-scope stores, complete before the
    // count), then the last of the S workgroups of this group sums them
    float* pg = a.part + ((size_t)g * a.S + s) * NPW * 256;
#pragma unroll
    for (int j = 0; j < NPW; ++j)
      __hip_atomic_store(pg + j * 256 + tid, v[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores have completed
    __syncthreads();
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(a.cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == (unsigned)(a.S - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;
    // all S partials in flight together (device-scope round trips), then
    // summed in split order
    const float* pb = a.part + (size_t)g * a.S * NPW * 256;
    float pv[BG_SMAX][NPW];
#pragma unroll
    for (int ss = 0; ss < BG_SMAX; ++ss)
#pragma unroll
      for (int j = 0; j < NPW; ++j)
        pv[ss][j] = ss < a.S ? __hip_atomic_load(pb + ((size_t)ss * NPW + j) * 256 + tid, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : 0.f;
#pragma unroll
    for (int j = 0; j < NPW; ++j) {
      float t = pv[0][j];
#pragma unroll
      for (int ss = 1; ss < BG_SMAX; ++ss)
        if (ss < a.S) t += pv[ss][j];
      v[j] = t;
    }
    if (tid == 0) __hip_atomic_store(a.cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int m = tid >> 4;
  float mean = 0.f, inv_std = 0.f;
  if constexpr (LNG) row_stats_merge(a, lnp, mean, inv_std);
  float y[NPW];
  bool valid[NPW];
#pragma unroll
  for (int j = 0; j < NPW; ++j) {
    const int n = (g * NPW + j) * 16 + (tid & 15);
    valid[j] = m < a.M && n < a.N;
    y[j] = 0.f;
    if (valid[j]) {
      float t = v[j];
      if constexpr (LNG) t = inv_std * (t - mean * a.ln_s[n]);
      y[j] = store_out(a, m, n, t);
    }
  }
  if (a.stats_part) row_stats_partial<NPW>(a, y, valid);
}

__global__ void row_stats_kernel(const float* __restrict__ x, int d, float* __restrict__ part) {
  // statistics partials of one group of width d per row (two passes as
  // layer_norm, gpt2.rs:636-666): part[m] = (mean, M2); one wave per row
  const float* row = x + (size_t)blockIdx.x * d;
  const int lane = threadIdx.x;
  float s = 0.f;
  for (int k = lane; k < d; k += 64) s += row[k];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / (float)d;
  float q = 0.f;
  for (int k = lane; k < d; k += 64) {
    const float t = row[k] - mean;
    q += t * t;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
  if (lane == 0) {
    part[2 * blockIdx.x] = mean;
    part[2 * blockIdx.x + 1] = q;
  }
}

}  // namespace

size_t tiled_weight_bytes(int N, int K, int wtype) {
  return (size_t)((N + 15) / 16) * 16 * (size_t)K * (wtype == W_F32 ? 4 : 2);
}

bool launch_tile_weights(hipStream_t s, const void* src, int wtype, int N, int K, void* dst) {
  const int TK = wtype == W_F32 ? 16 : 32;
  if (K % TK != 0) return false;
  const long nchunks = (long)((N + 15) / 16) * (K / TK) * 64;
  tile_weights_kernel<<<(unsigned)((nchunks + 255) / 256), 256, 0, s>>>(src, wtype, N, K, dst, nchunks);
  return hipGetLastError() == hipSuccess;
}

BgemvPlan bgemv_plan(int N, int K, int wtype, int npw_force, int s_force) {
  // Measured on MI355X over the GPT-2 decode shapes (2304..50257 rows, K 768..6400,
  // f32 and bf16): two panels per wave once there are >= 300 panels, one
  // below; the k range split over 4 workgroups for K >= 150 tiles, over 2 for
  // fewer than 120 panels (too few workgroups otherwise), else not at all.
  BgemvPlan pl{};
  const int TK = wtype == W_F32 ? 16 : 32;
  const int KT = K / TK, NP = (N + 15) / 16;
  pl.npw = npw_force > 0 ? npw_force : (NP >= 300 ? 2 : 1);
  int S = s_force > 0 ? s_force : (KT >= 150 ? 4 : (NP < 120 ? 2 : 1));
  if (S < 1) S = 1;
  if (S > BG_SMAX) S = BG_SMAX;
  pl.ktc = (KT + S * BG_NW - 1) / (S * BG_NW);
  // every workgroup must own at least one tile so that all S arrive
  while (S > 1 && (S - 1) * BG_NW * pl.ktc >= KT) {
    --S;
    pl.ktc = (KT + S * BG_NW - 1) / (S * BG_NW);
  }
  pl.S = S;
  pl.groups = (NP + pl.npw - 1) / pl.npw;
  return pl;
}

size_t bgemv_work_floats(const BgemvPlan& pl) { return pl.S > 1 ? (size_t)pl.groups * pl.S * pl.npw * 256 : 0; }

bool launch_bgemv(hipStream_t s, const BgemvPlan& pl, BgemvArgs a) {
  const int TK = a.wtype == W_F32 ? 16 : 32;
  if (a.M < 1 || a.M > 16 || a.K % TK != 0 || a.ldx % 4 != 0) return false;
  if (pl.S > BG_SMAX || (pl.S > 1 && (!a.part || !a.cnt))) return false;
  if (a.ln_g && (!a.ln_s || !a.ln_part || a.ln_groups < 1 || a.ln_groups > 16 * BG_LNG_PER || a.ln_cols < 1 ||
                 (a.ln_groups - 1) * a.ln_cols >= a.K || a.ln_groups * a.ln_cols < a.K))
    return false;
  if (a.stats_part && a.epi != EPI_BIAS_RESID) return false;
  a.S = pl.S;
  a.ktc = pl.ktc;
  const dim3 grid(pl.groups, pl.S);
  const dim3 block(64 * BG_NW);
#define BG_LAUNCH(WT, NPW)                                   \
  do {                                                       \
    if (a.ln_g) bgemv_kernel<WT, NPW, true><<<grid, block, 0, s>>>(a); \
    else bgemv_kernel<WT, NPW, false><<<grid, block, 0, s>>>(a);       \
  } while (0)
  if (a.wtype == W_F32) {
    if (pl.npw == 1) BG_LAUNCH(W_F32, 1);
    else if (pl.npw == 2) BG_LAUNCH(W_F32, 2);
    else BG_LAUNCH(W_F32, 4);
  } else {
    if (pl.npw == 1) BG_LAUNCH(W_BF16, 1);
    else if (pl.npw == 2) BG_LAUNCH(W_BF16, 2);
    else BG_LAUNCH(W_BF16, 4);
  }
#undef BG_LAUNCH
  return hipGetLastError() == hipSuccess;
}

void launch_row_stats(hipStream_t s, const float* x, int rows, int d, float* part) {
  row_stats_kernel<<<rows, 64, 0, s>>>(x, d, part);
}

}  // namespace rtg
