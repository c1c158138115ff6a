// Persistent batched decode step (2..16 sequences): one cooperative launch
// of 256 workgroups x 8 waves runs a whole decode step, phase by phase, with a
// grid barrier between phases instead of a kernel boundary:
//   embedding (+ LayerNorm statistics of the rows)       gpt2.rs:377-384
//   per layer: c_attn GEMV with LN1 folded, k/v into the cache;
//              attention over the cache;                  gpt2.rs:477-538
//              attn c_proj + residual (statistics partials);
//              c_fc GEMV with LN2 folded + gelu_new;
//              mlp c_proj + residual (statistics partials)
//   LM head with ln_f folded and the greedy argmax keys   gpt2.rs:392-396, 858-868
//   the last workgroup to finish writes the tokens, the ids and the counters
//   (the finalize of the reference loop, gpt2.rs:431-437).
// The GEMVs and the attention are the batched step's device functions
// (bgemv_core.h, attn_core.h) with device-scope (sc1) loads and stores for
// everything written within the launch. A phase's work units are spread over
// the workgroups round-robin.
//
// Barrier: each workgroup, after all its memory operations have completed,
// stores the phase's flag value into its own 128-byte slot; wave 0 polls all
// 256 slots (device-scope loads) until every value has reached it. Flag
// values only grow (the host advances bar_base by bd_barriers(L) per step).
// Every wait is bounded: a timeout sets *err and the step finishes with wrong
// numbers instead of hanging; the host turns *err into an error.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_core.h"
#include "bdecode.h"
#include "bgemv_core.h"

namespace rtg {

namespace {

constexpr int NW = 8, NT = 64 * NW;
constexpr unsigned BAR_SPIN_CAP = 1u << 20;

__device__ __forceinline__ bool err_set(const unsigned* err) {
  return __hip_atomic_load(const_cast<unsigned*>(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}

__device__ __forceinline__ void trace_point(const BdParams& p, int idx) {
  if (p.trace && blockIdx.x == 0 && threadIdx.x == 0) p.trace[idx] = wall_clock64();
}

__device__ __forceinline__ void grid_barrier(const BdParams& p, unsigned target) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's loads, stores and atomics have completed
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    if (lane == 0) __hip_atomic_store(p.bar + blockIdx.x * 32, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned spins = 0;
    for (;;) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < BD_G / 64; ++k) {
        const unsigned v = __hip_atomic_load(p.bar + (lane + 64 * k) * 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = ok && (int)(v - target) >= 0;
      }
      if (__all(ok)) break;
      if (++spins > BAR_SPIN_CAP || ((spins & 255u) == 0u && err_set(p.err))) {
        if (lane == 0) __hip_atomic_fetch_or(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  trace_point(p, (int)(target - p.bar_base));
}

// Sum over the workgroup in a fixed order (wave sums, then the waves in order).
__device__ __forceinline__ float block_sum(float v, float* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float t = scratch[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

template <int WT, int NPW, bool LNG>
__device__ __forceinline__ void gemv_phase(const BgemvArgs& a, const BgemvPlan& pl, float* red, unsigned* last) {
  const int U = pl.groups * pl.S;
  // a wave's whole k-chunk in flight at once when it has at most 8 tiles
  if (pl.ktc <= 8) {
    for (int u = blockIdx.x; u < U; u += BD_G)
      bgc::bgemv_unit<WT, NPW, LNG, NW, true, 8, true>(a, u / pl.S, u % pl.S,
                                                       reinterpret_cast<float(*)[NPW][256]>(red), last);
  } else {
    for (int u = blockIdx.x; u < U; u += BD_G)
      bgc::bgemv_unit<WT, NPW, LNG, NW, true>(a, u / pl.S, u % pl.S, reinterpret_cast<float(*)[NPW][256]>(red),
                                              last);
  }
}

template <int WT, bool LNG>
__device__ __forceinline__ void gemv_phase_npw(BgemvArgs a, const BgemvPlan& pl, float* red, unsigned* last) {
  a.S = pl.S;
  a.ktc = pl.ktc;
  if (pl.npw == 1) gemv_phase<WT, 1, LNG>(a, pl, red, last);
  else gemv_phase<WT, 2, LNG>(a, pl, red, last);
}

template <int WT>
__global__ __launch_bounds__(NT) void bdecode_kernel(BdParams p) {
  __shared__ float red[NW * 2 * 256];
  __shared__ float wp[NW][AD_ITEM];
  __shared__ float scratch[NW];
  __shared__ unsigned last;
  const int tid = threadIdx.x;
  const int d = p.d, B = p.B;
  const int pos = *p.pos;  // written by the previous step (kernel boundary)
  const int len = pos + 1;
  unsigned bar = p.bar_base;
  trace_point(p, 0);
  auto base = [&]() {
    BgemvArgs a{};
    a.M = B;
    a.wtype = WT;
    a.part = p.part;
    a.cnt = p.cnt;
    a.eps = p.eps;
    return a;
  };
  // ---- embedding + the rows' LayerNorm statistics (one group of width d) ----
  if ((int)blockIdx.x < B) {
    const int b = blockIdx.x;
    const long tok = p.token[b];
    float v[4];  // d <= 2048
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = tid + NT * i;
      v[i] = 0.f;
      if (k < d) {
        const float w = WT == W_F32 ? static_cast<const float*>(p.wte)[tok * d + k]
                                    : __uint_as_float((uint32_t)static_cast<const uint16_t*>(p.wte)[tok * d + k] << 16);
        v[i] = w + p.wpe[(long)pos * d + k];
        bgc::st1<true>(p.x + (long)b * d + k, v[i]);
        s += v[i];
      }
    }
    const float mean = block_sum(s, scratch) / (float)d;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t = v[i] - mean;
      q += tid + NT * i < d ? t * t : 0.f;
    }
    q = block_sum(q, scratch);
    if (tid == 0) {
      bgc::st1<true>(p.spart + 2 * b, mean);
      bgc::st1<true>(p.spart + 2 * b + 1, q);
    }
  }
  grid_barrier(p, ++bar);
  int st_groups = 1, st_cols = d;  // shape of the statistics partials of x
  for (int l = 0; l < p.L; ++l) {
    const BdLayer& T = p.layers[l];
    KvDst kv;
    kv.k = p.kc + (long)l * p.kv_layer;
    kv.v = p.vc + (long)l * p.kv_layer;
    kv.n_head = p.H;
    kv.n_pos = p.P;
    kv.d = d;
    {  // LN1 + c_attn; k/v of the new token into the cache
      BgemvArgs a = base();
      a.X = p.x; a.ldx = d; a.Wt = T.qkv; a.N = 3 * d; a.K = d; a.bias = T.cq;
      a.ln_g = T.ln1w; a.ln_s = T.sq; a.ln_part = p.spart; a.ln_groups = st_groups; a.ln_cols = st_cols;
      a.epi = EPI_BIAS;
      a.qkv = BgemvQkv{p.qkv, d, d, kv, p.pos};
      gemv_phase_npw<WT, true>(a, p.plan.pq, red, &last);
    }
    grid_barrier(p, ++bar);
    for (int it = blockIdx.x; it < B * p.H; it += BD_G)
      attn_item<NW, true>(p.qkv, d, kv.k, kv.v, p.H, p.P, len, it % p.H, it / p.H, p.att, d, wp);
    grid_barrier(p, ++bar);
    {  // attention c_proj + residual; statistics partials for LN2
      BgemvArgs a = base();
      a.X = p.att; a.ldx = d; a.Wt = T.proj; a.N = d; a.K = d; a.bias = T.baproj;
      a.C = p.x; a.ldc = d; a.epi = EPI_BIAS_RESID; a.stats_part = p.spart;
      gemv_phase_npw<WT, false>(a, p.plan.pp, red, &last);
      st_groups = p.plan.pp.groups;
      st_cols = 16 * p.plan.pp.npw;
    }
    grid_barrier(p, ++bar);
    {  // LN2 + c_fc + gelu_new
      BgemvArgs a = base();
      a.X = p.x; a.ldx = d; a.Wt = T.fc; a.N = 4 * d; a.K = d; a.bias = T.cf;
      a.ln_g = T.ln2w; a.ln_s = T.sf; a.ln_part = p.spart; a.ln_groups = st_groups; a.ln_cols = st_cols;
      a.C = p.h; a.ldc = 4 * d; a.epi = EPI_BIAS_GELU;
      gemv_phase_npw<WT, true>(a, p.plan.pf, red, &last);
    }
    grid_barrier(p, ++bar);
    {  // mlp c_proj + residual; statistics partials for the next LayerNorm
      BgemvArgs a = base();
      a.X = p.h; a.ldx = 4 * d; a.Wt = T.mproj; a.N = d; a.K = 4 * d; a.bias = T.bmproj;
      a.C = p.x; a.ldc = d; a.epi = EPI_BIAS_RESID; a.stats_part = p.spart;
      gemv_phase_npw<WT, false>(a, p.plan.pm, red, &last);
      st_groups = p.plan.pm.groups;
      st_cols = 16 * p.plan.pm.npw;
    }
    grid_barrier(p, ++bar);
  }
  {  // ln_f + tied LM head + argmax keys
    BgemvArgs a = base();
    a.X = p.x; a.ldx = d; a.Wt = p.lm; a.N = p.V; a.K = d; a.bias = p.cl;
    a.ln_g = p.lnfw; a.ln_s = p.sl; a.ln_part = p.spart; a.ln_groups = st_groups; a.ln_cols = st_cols;
    a.C = p.logits; a.ldc = p.V; a.epi = EPI_BIAS; a.keys = p.keys;
    gemv_phase_npw<WT, true>(a, p.plan.pl, red, &last);
  }
  trace_point(p, bd_barriers(p.L) + 1);
  // The last workgroup to arrive (its key updates and everyone else's have
  // completed: each counts itself only after its own have) finishes the step.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const unsigned arrived = __hip_atomic_fetch_add(p.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == BD_G - 1) {
      const int step = *p.step;
      for (int b = 0; b < B; ++b) {
        const unsigned long long key =
            __hip_atomic_load(p.keys + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t next = argmax_key_index(key);
        p.token[b] = next;
        p.ids[(long)b * p.ld_ids + step] = next;
        __hip_atomic_store(p.keys + b, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *p.pos = pos + 1;
      *p.step = step + 1;
      __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

BgemvPlan bd_plan(int N, int K, int wtype) {
  // Rounds of units per workgroup times the tiles of a wave in a unit plus a
  // fixed cost per unit, plus the split-k fix-up: the cheapest (npw, S).
  BgemvPlan best{};
  long best_cost = -1;
  for (int npw = 1; npw <= 2; ++npw)
    for (int S = 1; S <= 8; S *= 2) {
      BgemvPlan pl = bgemv_plan(N, K, wtype, npw, S, NW);
      const long units = (long)pl.groups * pl.S;
      const long rounds = (units + BD_G - 1) / BD_G;
      const long cost = rounds * (npw * pl.ktc + 4) + (pl.S > 1 ? 6 : 0);
      if (best_cost < 0 || cost < best_cost) {
        best_cost = cost;
        best = pl;
      }
    }
  return best;
}

size_t bd_part_floats(const BdPlans& p) {
  size_t m = 1;
  for (const BgemvPlan* pl : {&p.pq, &p.pp, &p.pf, &p.pm, &p.pl}) {
    const size_t f = bgemv_work_floats(*pl);
    m = f > m ? f : m;
  }
  return m;
}

size_t bd_groups(const BdPlans& p) {
  size_t m = 1;
  for (const BgemvPlan* pl : {&p.pq, &p.pp, &p.pf, &p.pm, &p.pl}) m = (size_t)pl->groups > m ? pl->groups : m;
  return m;
}

hipError_t launch_bdecode(const BdParams& p, hipStream_t s) {
  if (p.B < 1 || p.B > 16 || p.d > 2048 || p.d % 64 != 0 || p.H * 64 != p.d) return hipErrorInvalidValue;
  void* args[] = {const_cast<BdParams*>(&p)};
  const void* fn = p.wtype == W_F32 ? (const void*)bdecode_kernel<W_F32> : (const void*)bdecode_kernel<W_BF16>;
  return hipLaunchCooperativeKernel(fn, dim3(BD_G), dim3(NT), args, 0, s);
}

}  // namespace rtg
