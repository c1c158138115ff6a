// Token choice on the device: sample_logits (rusttorch-core/src/nn/gpt2.rs:
// 871-906) with repetition penalty (:909-921), temperature, top-k (:924-935),
// top-p (:939-970) and sample_from_logits (:973-993); the greedy branch with a
// repetition penalty (:872-880); and sample_with_temperature (:996-1017),
// which is sample_logits without penalty and filters.
//
// One workgroup of 512 threads per sequence. Element i is held in a register
// of thread i % 512 (row i / 512: the row index is the register index, so
// the load is one coalesced sweep and every later pass works on registers).
// Questions in index order (the sampling CDF, the order of top-p ties) are
// answered from per-(row, wave) partial sums kept in LDS. The repetition
// penalty edits a copy of the logits in device memory before the load.
//
// The uniform draw of generation index g is output number draw0 + g + 1 of
// SplitMix64 seeded with the caller's seed, mix(seed + k * 0x9E3779B97F4A7C15),
// as 24 bits / 2^24: the sequence of the host sampler (the reference draws
// from rand::thread_rng, so its samples are not reproducible at all).
//
// Sums (softmax denominators, top-p masses, the CDF) are formed in a fixed
// order, so results are deterministic, but not in the reference's sequential
// order: a draw within rounding distance of a CDF boundary can pick the
// neighbouring token.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace rtg {
namespace {

constexpr int ST = 512;        // threads (2 waves per SIMD: up to 256 registers each)
constexpr int SW = ST / 64;    // waves
constexpr int MAX_ROWS = 128;  // V <= 65536

__device__ __forceinline__ float wave_sum_s(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_s(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

struct SampleSmem {
  float red[SW];
  float seg[MAX_ROWS * SW];      // per (row, wave) values, index order
  float segpre[MAX_ROWS * SW];   // their exclusive prefix sums
  unsigned hist[256];
  unsigned mass[256];  // fixed-point probability mass per digit
  unsigned long long key;
  uint32_t hist_tokens[ST];
  unsigned misc[8];
  unsigned long long lmisc[2];
  float fmisc[2];
};

// Sum / max over the block in a fixed order; every thread gets the result.
__device__ float block_sum(float v, SampleSmem& sm) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  v = wave_sum_s(v);
  __syncthreads();
  if (l == 0) sm.red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < SW; ++i) t += sm.red[i];
  return t;
}
__device__ float block_max(float v, SampleSmem& sm) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  v = wave_max_s(v);
  __syncthreads();
  if (l == 0) sm.red[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < SW; ++i) t = fmaxf(t, sm.red[i]);
  return t;
}

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t k) {
  uint64_t z = seed + k * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Lanes below this one whose bit is set in a wave ballot.
__device__ __forceinline__ int lanes_before(unsigned long long ballot) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(ballot >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ballot, 0u));
}

// Wave 0 only: the largest bin b (of 256, counts or fixed-point masses h)
// whose running total from the top, sum_{b' >= b} h[b'], reaches need, and the
// total of the bins above it. Returns -1 when the bins do not reach need.
template <typename T>
__device__ int wave_top_bin(const T* h, T need, int lane, T* above_out) {
  T v[4], s = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // lane l: bins 255 - 4l - k, descending
    v[k] = h[255 - 4 * lane - k];
    s += v[k];
  }
  T incl = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  T cum = incl - s;
  int found = -1;
  T above = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (found < 0 && cum + v[k] >= need) {
      found = 255 - 4 * lane - k;
      above = cum;
    }
    cum += v[k];
  }
  const unsigned long long bal = __ballot(found >= 0);
  if (!bal) return -1;
  const int src = __builtin_ctzll(bal);
  *above_out = __shfl(above, src, 64);
  return __shfl(found, src, 64);
}

// Wave 0 only: segpre[i] = sum of seg[0, i) for i < n (n <= 64 * 16), each
// lane summing a contiguous run in order, then the runs' prefix.
__device__ void wave_excl_prefix(const float* seg, float* segpre, int n, int lane) {
  const int per = (n + 63) / 64, b = lane * per, e = min(n, b + per);
  float s = 0.f;
  for (int i = b; i < e; ++i) s += seg[i];
  float incl = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  float run = incl - s;
  for (int i = b; i < e; ++i) {
    segpre[i] = run;
    run += seg[i];
  }
}

__device__ __forceinline__ uint32_t hist_at(const uint32_t* prompt, int n_prompt, const uint32_t* ids, int q) {
  return q < n_prompt ? prompt[q] : ids[q - n_prompt];
}

}  // namespace

template <int NJ>
__global__ __launch_bounds__(ST) void sample_kernel(const float* __restrict__ logits, int V, float* __restrict__ work,
                                                    const uint32_t* __restrict__ prompt, int n_prompt,
                                                    uint32_t* __restrict__ ids, const int* __restrict__ step_dev,
                                                    SampleParams sp, uint32_t* __restrict__ token) {
  __shared__ SampleSmem sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = *step_dev - 1;  // generation index of the token being chosen
  // v[j] = element j * ST + t ("row" j), in registers for all passes
  float v[NJ];
  const float* src = logits;
  // ---- repetition penalty over prompt + generated tokens (gpt2.rs:909-921):
  // once per occurrence; the first occurrence of a token in the history
  // applies all of its occurrences, one after the other, to a copy in memory ----
  if (sp.penalty != 1.0f) {
    for (int i = t; i < V; i += ST) work[i] = logits[i];
    const int nh = n_prompt + g;
    for (int base = 0; base < nh; base += ST) {
      __syncthreads();
      if (base + t < nh) sm.hist_tokens[t] = hist_at(prompt, n_prompt, ids, base + t);
      __syncthreads();
      const int cnt = min(ST, nh - base);
      if (t < cnt) {
        const uint32_t tok = sm.hist_tokens[t];
        bool first = true;
        for (int q = 0; q < base && first; ++q) first = hist_at(prompt, n_prompt, ids, q) != tok;
        for (int q = 0; q < t && first; ++q) first = sm.hist_tokens[q] != tok;
        if (first && tok < (uint32_t)V) {
          int c = 1;
          for (int q = t + 1; q < cnt; ++q) c += sm.hist_tokens[q] == tok;
          for (int q = base + ST; q < nh; ++q) c += hist_at(prompt, n_prompt, ids, q) == tok;
          float x = work[tok];
          for (int k = 0; k < c; ++k) x = x > 0.0f ? x / sp.penalty : x * sp.penalty;
          work[tok] = x;
        }
      }
    }
    __syncthreads();
    src = work;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = j * ST + t;
    v[j] = i < V ? src[i] : -INFINITY;
  }
  uint32_t pick = 0;
  if (sp.temperature <= 0.0f) {
    // ---- greedy: argmax_f32 (gpt2.rs:858-868), strict '>' from -inf, the
    // first index wins, NaN never wins ----
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = j * ST + t;
      if (i < V && v[j] > -INFINITY) {
        const unsigned long long k = ((unsigned long long)order_key(v[j]) << 32) | (uint32_t)~(uint32_t)i;
        best = k > best ? k : best;
      }
    }
    if (t == 0) sm.key = 0ull;
    __syncthreads();
    if (best) atomicMax(&sm.key, best);
    __syncthreads();
    pick = sm.key ? ~(uint32_t)(sm.key & 0xffffffffull) : 0u;
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = v[j] / sp.temperature;
    // ---- top-k (gpt2.rs:924-935): threshold = k-th largest value, found
    // exactly by an 8-bit radix select on order-preserving keys ----
    if (sp.top_k > 0 && sp.top_k < V) {
      uint32_t prefix = 0, need = (uint32_t)sp.top_k;
      for (int shift = 24; shift >= 0; shift -= 8) {
        const uint32_t hi_mask = shift == 24 ? 0u : ~((1u << (shift + 8)) - 1u);
        if (t < 256) sm.hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t k = order_key(v[j]);
          if (j * ST + t < V && (k & hi_mask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (w == 0) {
          unsigned above = 0;
          const int b = wave_top_bin<unsigned>(sm.hist, need, lane, &above);
          if (lane == 0) {
            sm.misc[0] = (uint32_t)max(b, 0);  // need <= the count in range: b >= 0
            sm.misc[1] = need - above;
          }
        }
        __syncthreads();
        prefix |= sm.misc[0] << shift;
        need = sm.misc[1];
        __syncthreads();
      }
      const float thr = from_order_key(prefix);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (v[j] < thr) v[j] = -INFINITY;
    }
    // From here v holds the probabilities p = exp(x - max) / sum of the
    // filtered logits x (0 for the removed ones). Top-p keeps the largest
    // probability, so the maximum of what it leaves is the same, and the
    // distribution sample_from_logits draws from is p / (kept mass): top-p
    // zeroes entries in place.
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NJ; ++j) mx = fmaxf(mx, v[j]);
    mx = block_max(mx, sm);
    float loc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      v[j] = j * ST + t < V ? expf(v[j] - mx) : 0.f;
      loc += v[j];
    }
    float sum = block_sum(loc, sm);
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = v[j] / sum;
    sum = 1.0f;  // mass of the kept entries, as a divisor of p
    // ---- top-p (gpt2.rs:939-970): keep the largest probabilities, ties in
    // index order, until their running sum reaches p ----
    if (sp.top_p < 1.0f && sp.top_p > 0.0f) {
      // radix descent (8-bit digits) over the bits of the probabilities
      // (non-negative floats order like their bits) for the cut-off value,
      // mass(p > cut) < top_p <= mass(p >= cut), with masses summed as
      // integers (p * 2^31, truncated; at most 2^-31 per entry): the same
      // total in any order.
      const float scale = 2147483648.0f;  // 2^31
      const unsigned target = (unsigned)(sp.top_p * scale);
      uint32_t prefix = 0;
      unsigned above = 0;
      bool all = false;
      for (int shift = 24; shift >= 0 && !all; shift -= 8) {
        const uint32_t hi_mask = shift == 24 ? 0u : ~((1u << (shift + 8)) - 1u);
        if (t < 256) sm.mass[t] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t k = __float_as_uint(v[j]);
          if (j * ST + t < V && (k & hi_mask) == prefix) atomicAdd(&sm.mass[(k >> shift) & 255u], (unsigned)(v[j] * scale));
        }
        __syncthreads();
        if (w == 0) {
          unsigned ab = 0;
          const int bin = wave_top_bin<unsigned>(sm.mass, target - above, lane, &ab);
          if (lane == 0) {
            sm.misc[0] = (unsigned)bin;
            sm.misc[1] = ab;
          }
        }
        __syncthreads();
        const int bin = (int)sm.misc[0];
        if (bin < 0) all = true;  // the total stays below p: everything is kept
        else {
          prefix |= (uint32_t)bin << shift;
          above += sm.misc[1];
        }
        __syncthreads();
      }
      if (!all) {
        // ties at the cut-off value, in index order: the first `take` are
        // kept, as many as the running sum needs to reach p
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bool tie = j * ST + t < V && __float_as_uint(v[j]) == prefix;
          const unsigned long long bal = __ballot(tie);
          if (lane == 0) sm.seg[j * SW + w] = (float)__popcll(bal);
        }
        __syncthreads();
        if (w == 0) {
          wave_excl_prefix(sm.seg, sm.segpre, NJ * SW, lane);
          if (lane == 0) {
            const unsigned qcut = (unsigned)(__uint_as_float(prefix) * scale);
            sm.misc[2] = qcut ? (target - above + qcut - 1) / qcut : 0xffffffffu;
          }
        }
        __syncthreads();
        const unsigned take = sm.misc[2];
        loc = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t k = __float_as_uint(v[j]);
          const bool tie = j * ST + t < V && k == prefix;
          const unsigned long long bal = __ballot(tie);
          bool keep = k > prefix;
          if (tie) keep = (unsigned)sm.segpre[j * SW + w] + (unsigned)lanes_before(bal) < take;
          if (!keep) v[j] = 0.f;
          loc += v[j];
        }
        sum = block_sum(loc, sm);
      }
    }
    // ---- sample_from_logits (gpt2.rs:973-993): the first index whose
    // running sum of probabilities exceeds the uniform draw ----
    const float r = (float)(splitmix_at(sp.seed, (uint64_t)sp.draw0 + (uint64_t)g + 1) >> 40) * (1.0f / 16777216.0f);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      v[j] = v[j] / sum;
      const float ws = wave_sum_s(v[j]);
      if (lane == 0) sm.seg[j * SW + w] = ws;
    }
    __syncthreads();
    if (w == 0) {
      // the (row, wave) segment of 64 indices where the running sum first exceeds r
      const int n = NJ * SW;
      wave_excl_prefix(sm.seg, sm.segpre, n, lane);
      const int per = (n + 63) / 64, b0 = lane * per, e0 = min(n, b0 + per);
      int found = -1;
      for (int i = b0; i < e0 && found < 0; ++i)
        if (r < sm.segpre[i] + sm.seg[i]) found = i;
      const unsigned long long bal = __ballot(found >= 0);
      const int segi = bal ? __shfl(found, __builtin_ctzll(bal), 64) : -1;
      if (lane == 0) {
        sm.misc[3] = segi < 0 ? 0xffffffffu : (unsigned)segi;
        sm.fmisc[0] = segi < 0 ? 0.f : sm.segpre[segi];
      }
    }
    __syncthreads();
    const unsigned seg = sm.misc[3];
    if (seg == 0xffffffffu) {
      pick = (uint32_t)(V - 1);
    } else {
      // inside the segment: 64 consecutive indices, held by wave seg % SW in row seg / SW
      if (w == (int)(seg % SW)) {
        const int row = (int)(seg / SW);
        float p = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          if (j == row) p = v[j];
        const int i = row * ST + t;
        float incl = p;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const float u = __shfl_up(incl, o, 64);
          if (lane >= o) incl += u;
        }
        const unsigned long long bal = __ballot(i < V && r < sm.fmisc[0] + incl);
        // the segment's sum (a tree) put r inside it; should the running sum
        // (another order) stop short by rounding, the segment's last index of
        // non-zero probability is the one the draw falls on
        const unsigned long long nz = __ballot(i < V && p > 0.f);
        const int i0 = row * ST + (int)(seg % SW) * 64;
        if (lane == 0)
          sm.misc[4] = bal ? (unsigned)(i0 + __builtin_ctzll(bal))
                           : nz ? (unsigned)(i0 + 63 - __builtin_clzll(nz)) : (unsigned)(V - 1);
      }
      __syncthreads();
      pick = sm.misc[4];
    }
  }
  if (t == 0) {
    token[0] = pick;
    ids[g] = pick;
  }
}

bool launch_sample(hipStream_t s, const float* logits, int V, float* work, const uint32_t* prompt, int n_prompt,
                   uint32_t* ids, const int* step_dev, const SampleParams& sp, uint32_t* token) {
#define RTG_SAMPLE(NJ) sample_kernel<NJ><<<1, ST, 0, s>>>(logits, V, work, prompt, n_prompt, ids, step_dev, sp, token)
  if (V <= 0) return false;
  if (V <= 1 * ST) RTG_SAMPLE(1);
  else if (V <= 4 * ST) RTG_SAMPLE(4);
  else if (V <= 16 * ST) RTG_SAMPLE(16);
  else if (V <= 64 * ST) RTG_SAMPLE(64);
  else if (V <= 100 * ST) RTG_SAMPLE(100);  // GPT-2's 50257 tokens
  else if (V <= 128 * ST) RTG_SAMPLE(128);
  else return false;
#undef RTG_SAMPLE
  return true;
}

}  // namespace rtg
