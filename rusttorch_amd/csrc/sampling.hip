// Token choice on the device: sample_logits (rusttorch-core/src/nn/gpt2.rs:
// 871-906) with repetition penalty (:909-921), temperature, top-k (:924-935),
// top-p (:939-970) and sample_from_logits (:973-993); the greedy branch with a
// repetition penalty (:872-880); and sample_with_temperature (:996-1017),
// which is sample_logits without penalty and filters.
//
// One workgroup of 512 threads per sequence. Element i is held in a register
// of thread i % 512 (row i / 512: the row index is the register index, so
// the load is one coalesced sweep and every later pass works on registers).
// The work is VALU-bound on the one CU, so every pass over the row is kept to
// a few instructions per element:
//  - the repetition penalty marks the history in an LDS bitmap and counts it
//    in an LDS hash table; each element tests its bit and, when set, applies
//    the penalty once per occurrence to its register;
//  - top-k and top-p find their cut-off by histogram rounds (radix select).
//    The first round of top-k bins the scaled logits linearly (2048 bins)
//    between their minimum and maximum, the first round of top-p bins the exponent and two
//    mantissa bits of exp(y - max): both spread the values over many bins, so
//    the LDS atomics rarely collide, and both maps are monotone, so the bin of
//    the k-th value (of the mass crossing p) is exact. Later rounds refine the
//    key bits of that bin's members only;
//  - questions in index order (the sampling CDF, the order of top-p ties) are
//    answered from per-(row, wave) partial sums, reduced across the wave by a
//    transposing butterfly (one shuffle per row and stage, halving the rows at
//    each stage).
//
// The uniform draw of generation index g is output number draw0 + g + 1 of
// SplitMix64 seeded with the caller's seed, mix(seed + k * 0x9E3779B97F4A7C15),
// as 24 bits / 2^24: the sequence of the host sampler (the reference draws
// from rand::thread_rng, so its samples are not reproducible at all).
//
// Sums (softmax denominators, top-p masses, the CDF) are formed in a fixed
// order, so results are deterministic, but not in the reference's sequential
// order, and the CDF is compared in unnormalised form (draw * total against
// running sums of exp(y - max)): a draw within rounding distance of a CDF
// boundary can pick the neighbouring token.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "argmax_key.h"
#include "kernels.h"

namespace rtg {
namespace {

constexpr int ST = 512;        // threads (2 waves per SIMD: up to 256 registers each)
constexpr int SW = ST / 64;    // waves
constexpr int MAX_ROWS = 128;  // V <= 65536
constexpr int NB = 2048;       // histogram bins of the widest round (11 bits)
constexpr int PBW = MAX_ROWS * ST / 32;  // words of the token bitmap
constexpr int DMAX = 2048;  // distinct penalised tokens per penalty round
constexpr uint32_t NONE = 0xffffffffu;

__device__ __forceinline__ float wave_max_s(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_min_s(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}

struct SampleSmem {
  float red[2 * SW];
  unsigned wtot[SW];
  union {
    struct {                        // selection and the draw
      unsigned hist[NB];            // counts or fixed-point probability masses per bin
      float seg[MAX_ROWS * SW];     // per (row, wave) values, index order
      float segpre[MAX_ROWS * SW];  // their exclusive prefix sums
    };
    struct {                  // repetition penalty
      uint32_t wordpre[PBW];  // marked tokens in the bitmap words before each word
      uint32_t cnt[DMAX];     // occurrences per marked token, by rank
      float val[DMAX];        // penalised logit per marked token, by rank
    };
  };
  uint32_t pbits[PBW];  // tokens of the history (within the round's range)
  unsigned misc[8];
  unsigned long long key;
  float fmisc[2];
};

// Max / min over the block in a fixed order; every thread gets the result.
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
__device__ void block_minmax(float& mx, float& mn, SampleSmem& sm) {
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  mx = wave_max_s(mx);
  mn = wave_min_s(mn);
  __syncthreads();
  if (l == 0) {
    sm.red[w] = mx;
    sm.red[SW + w] = mn;
  }
  __syncthreads();
  mx = -INFINITY;
  mn = INFINITY;
  for (int i = 0; i < SW; ++i) {
    mx = fmaxf(mx, sm.red[i]);
    mn = fminf(mn, sm.red[SW + i]);
  }
}

// Bin of y among NB linear bins from mn (scale bs = (NB - 1) / range, or 0):
// monotone in y; -inf and NaN go to bin 0.
__device__ __forceinline__ unsigned lin_bin(float y, float mn, float bs) {
  return (unsigned)fminf(fmaxf((y - mn) * bs, 0.f), (float)(NB - 1));
}

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Fixed-point probability mass of e (scale ms = 2^31 / sum): rounded to
// nearest, so the error of a sum over many entries stays unbiased (truncation
// would lose half a unit per entry: ~1e-5 over 45k kept entries, enough to
// move the top-p cut).
__device__ __forceinline__ unsigned mass_of(float e, float ms) { return (unsigned)(e * ms + 0.5f); }

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

// Exclusive prefix of x over the block in thread order; the total in *total.
__device__ unsigned block_excl_scan(unsigned x, SampleSmem& sm, unsigned* total) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  unsigned incl = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  __syncthreads();
  if (lane == 63) sm.wtot[w] = incl;
  __syncthreads();
  unsigned base = 0, tot = 0;
  for (int i = 0; i < SW; ++i) {
    if (i == w) base = tot;
    tot += sm.wtot[i];
  }
  *total = tot;
  return base + incl - x;
}

// Whole block, after the histogram h[NBINS] is complete: the largest bin b
// whose running total from the top, sum_{b' >= b} h[b'], reaches need (>= 1).
// Leaves b (NONE when the bins do not reach need), the total of the bins above
// it and h[b] in misc[0..2]; ends synchronised.
template <int NBINS>
__device__ void block_top_bin(const unsigned* h, unsigned need, SampleSmem& sm) {
  constexpr int BPT = NBINS / ST;
  static_assert(BPT * ST == NBINS, "bins per thread");
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  unsigned v[BPT], s = 0;
#pragma unroll
  for (int k = 0; k < BPT; ++k) {  // thread t: bins NBINS-1-BPT*t-k, descending
    v[k] = h[NBINS - 1 - BPT * t - k];
    s += v[k];
  }
  unsigned incl = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63) sm.wtot[w] = incl;
  if (t == 0) sm.misc[0] = NONE;
  __syncthreads();
  unsigned cum = incl - s;
  for (int i = 0; i < w; ++i) cum += sm.wtot[i];
  // running totals only grow: exactly one thread sees need crossed in its bins
  if (cum < need && need <= cum + s) {
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      if (cum < need && need <= cum + v[k]) {
        sm.misc[0] = (unsigned)(NBINS - 1 - BPT * t - k);
        sm.misc[1] = cum;
        sm.misc[2] = v[k];
      }
      cum += v[k];
    }
  }
  __syncthreads();
}

// A histogram round: hist_begin clears NBINS bins; the caller accumulates;
// hist_end finds the top bin reaching need (results in misc[0..2] for every
// thread).
template <int NBINS>
__device__ __forceinline__ void hist_begin(SampleSmem& sm) {
  for (int b = threadIdx.x; b < NBINS; b += ST) sm.hist[b] = 0u;
  __syncthreads();
}
template <int NBINS>
__device__ __forceinline__ void hist_end(SampleSmem& sm, unsigned need) {
  __syncthreads();
  block_top_bin<NBINS>(sm.hist, need, sm);
}

// Wave 0 only: segpre[i] = sum of seg[0, i) for i < n (n <= 64 * 16), each
// lane summing a contiguous run in order, then the runs' prefix. Returns the
// total to every lane.
__device__ float wave_excl_prefix(const float* seg, float* segpre, int n, int lane) {
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
  return __shfl(incl, 63, 64);
}

// One stage of the transposing butterfly over 16-row chunks: N values per
// lane become N/2; the lane with bit O set keeps the upper half.
template <int N, int O>
__device__ __forceinline__ void tr_stage(float (&a)[16], int lane) {
  constexpr int H = N / 2;
  const bool up = (lane & O) != 0;
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const float send = up ? a[k] : a[k + H];
    const float keep = up ? a[k + H] : a[k];
    a[k] = keep + __shfl_xor(send, O, 64);
  }
}

// seg[row * SW + w] = sum of the wave's 64 values of each row (the 64
// consecutive indices row * ST + w * 64 ...). After the four halving stages
// lane l holds row (l >> 2) of its 16-row chunk, summed over its lane group;
// two butterflies finish the sum.
template <int NJ>
__device__ __forceinline__ void seg_sums(const float (&v)[NJ], float* seg, int w, int lane) {
#pragma unroll
  for (int c0 = 0; c0 < NJ; c0 += 16) {
    float a[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) a[k] = c0 + k < NJ ? v[c0 + k] : 0.f;
    tr_stage<16, 32>(a, lane);
    tr_stage<8, 16>(a, lane);
    tr_stage<4, 8>(a, lane);
    tr_stage<2, 4>(a, lane);
    a[0] += __shfl_xor(a[0], 2, 64);
    a[0] += __shfl_xor(a[0], 1, 64);
    const int r = c0 + (lane >> 2);
    if ((lane & 3) == 0 && r < NJ) seg[r * SW + w] = a[0];
  }
}

// Segment sums of v and their prefix (seg, segpre); returns the total.
template <int NJ>
__device__ __forceinline__ float seg_total(const float (&v)[NJ], SampleSmem& sm, int w, int lane) {
  seg_sums<NJ>(v, sm.seg, w, lane);
  __syncthreads();
  if (w == 0) {
    const float tot = wave_excl_prefix(sm.seg, sm.segpre, NJ * SW, lane);
    if (lane == 0) sm.fmisc[1] = tot;
  }
  __syncthreads();
  return sm.fmisc[1];
}

__device__ __forceinline__ uint32_t hist_at(const uint32_t* prompt, int n_prompt, const uint32_t* ids, int q) {
  return q < n_prompt ? prompt[q] : ids[q - n_prompt];
}

// Dense rank of a marked token: marked tokens below it.
__device__ __forceinline__ unsigned mark_rank(const SampleSmem& sm, uint32_t tok) {
  return sm.wordpre[tok >> 5] + (unsigned)__popc(sm.pbits[tok >> 5] & ((1u << (tok & 31u)) - 1u));
}

// gpt2.rs:909-921: for every token of the history (prompt and generated),
// logit /= penalty if it is positive, else logit *= penalty, once per
// occurrence. Per round of token ids (all of them at once while the history
// has at most DMAX entries): the history's tokens are marked in an LDS bitmap,
// the marks ranked densely (prefix popcounts of the words) and counted per
// rank; one thread per marked token applies its occurrences to the logit as
// loaded, and every element reads its result by rank.
template <int NJ>
__device__ __forceinline__ void apply_penalty(float (&v)[NJ], const float* logits, int V, const uint32_t* prompt,
                                              int n_prompt, const uint32_t* ids, int nh, float pen, SampleSmem& sm) {
  const int t = threadIdx.x;
  const int span = nh <= DMAX ? V : DMAX;  // token ids per round: at most DMAX marks
  constexpr int WPT = PBW / ST;            // bitmap words per thread in the scan
  for (int lo = 0; lo < V; lo += span) {
    const uint32_t hi = (uint32_t)min(V, lo + span);
    for (int i = t; i < PBW; i += ST) sm.pbits[i] = 0u;
    for (int i = t; i < DMAX; i += ST) sm.cnt[i] = 0u;
    __syncthreads();
    for (int q = t; q < nh; q += ST) {
      const uint32_t tok = hist_at(prompt, n_prompt, ids, q);
      if (tok >= (uint32_t)lo && tok < hi) atomicOr(&sm.pbits[tok >> 5], 1u << (tok & 31u));
    }
    __syncthreads();
    unsigned pc[WPT], s = 0, marks;
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
      pc[k] = (unsigned)__popc(sm.pbits[t * WPT + k]);
      s += pc[k];
    }
    unsigned run = block_excl_scan(s, sm, &marks);
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
      sm.wordpre[t * WPT + k] = run;
      run += pc[k];
    }
    __syncthreads();
    for (int q = t; q < nh; q += ST) {
      const uint32_t tok = hist_at(prompt, n_prompt, ids, q);
      if (tok >= (uint32_t)lo && tok < hi) atomicAdd(&sm.cnt[mark_rank(sm, tok)], 1u);
    }
    __syncthreads();
    for (unsigned r = t; r < marks; r += ST) {
      int a = 0, b = PBW - 1;  // the last word with wordpre <= r holds mark r
      while (a < b) {
        const int m = (a + b + 1) >> 1;
        if (sm.wordpre[m] <= r) a = m;
        else b = m - 1;
      }
      uint32_t word = sm.pbits[a];
      for (unsigned z = r - sm.wordpre[a]; z > 0; --z) word &= word - 1u;  // drop the lower marks
      float x = logits[a * 32 + __builtin_ctz(word)];
      for (unsigned z = sm.cnt[r]; z > 0; --z) x = x > 0.0f ? x / pen : x * pen;
      sm.val[r] = x;
    }
    __syncthreads();
    // element j * ST + t is bit t % 32 of word j * ST / 32 + t / 32
    const uint32_t below = (1u << (t & 31)) - 1u;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int wi = j * (ST / 32) + (t >> 5);
      const uint32_t word = sm.pbits[wi];
      if ((word >> (t & 31)) & 1u) v[j] = sm.val[sm.wordpre[wi] + (unsigned)__popc(word & below)];
    }
    __syncthreads();
  }
}

}  // namespace

template <int NJ>
__global__ __launch_bounds__(ST) void sample_kernel(const float* __restrict__ logits, int V,
                                                    const uint32_t* __restrict__ prompt, int n_prompt,
                                                    uint32_t* __restrict__ ids, const int* __restrict__ step_dev,
                                                    SampleParams sp, uint32_t* __restrict__ token) {
  __shared__ SampleSmem sm;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = *step_dev - 1;  // generation index of the token being chosen
  // v[j] = element j * ST + t ("row" j), in registers for all passes
  float v[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int i = j * ST + t;
    v[j] = i < V ? logits[i] : -INFINITY;
  }
  if (sp.penalty != 1.0f) apply_penalty<NJ>(v, logits, V, prompt, n_prompt, ids, n_prompt + g, sp.penalty, sm);
  uint32_t pick = 0;
  if (sp.temperature <= 0.0f) {
    // ---- greedy: argmax_f32 (gpt2.rs:858-868), strict '>' from -inf, the
    // first index wins, NaN never wins, -0.0 ties with +0.0 (argmax_key.h) ----
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int i = j * ST + t;
      if (i < V) {
        const unsigned long long k = argmax_key(v[j], (uint32_t)i);
        best = k > best ? k : best;
      }
    }
    if (t == 0) sm.key = 0ull;
    __syncthreads();
    if (best) atomicMax(&sm.key, best);
    __syncthreads();
    pick = argmax_key_index(sm.key);
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = v[j] / sp.temperature;
    float mx;
    if (sp.top_k > 0 && sp.top_k < V) {
      // ---- top-k (gpt2.rs:924-935): threshold = the k-th largest value ----
      float mn = INFINITY;
      mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (v[j] > -INFINITY) {
          mx = fmaxf(mx, v[j]);
          mn = fminf(mn, v[j]);
        }
      block_minmax(mx, mn, sm);
      // round 1: NB linear bins over [mn, mx]; a monotone map, so equal
      // values share a bin and every value in a higher bin is larger
      const float range = mx - mn;
      const float bs = (range > 0.f && range < INFINITY) ? (float)(NB - 1) / range : 0.f;
      hist_begin<NB>(sm);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (j * ST + t < V) atomicAdd(&sm.hist[lin_bin(v[j], mn, bs)], 1u);
      hist_end<NB>(sm, (unsigned)sp.top_k);
      const unsigned b1 = sm.misc[0];  // k < V elements: always found
      unsigned need = (unsigned)sp.top_k - sm.misc[1];
      uint32_t mm[(NJ + 31) / 32];  // members of bin b1
#pragma unroll
      for (int q = 0; q < (NJ + 31) / 32; ++q) mm[q] = 0u;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (j * ST + t < V && lin_bin(v[j], mn, bs) == b1) mm[j >> 5] |= 1u << (j & 31);
      // rounds 2-4: the order-preserving key of the members, 11 + 11 + 10 bits
      hist_begin<2048>(sm);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if ((mm[j >> 5] >> (j & 31)) & 1u) atomicAdd(&sm.hist[order_key(v[j]) >> 21], 1u);
      hist_end<2048>(sm, need);
      uint32_t prefix = sm.misc[0] << 21;
      need -= sm.misc[1];
      hist_begin<2048>(sm);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if ((mm[j >> 5] >> (j & 31)) & 1u) {
          const uint32_t k = order_key(v[j]);
          if ((k >> 21) == (prefix >> 21)) atomicAdd(&sm.hist[(k >> 10) & 2047u], 1u);
        }
      hist_end<2048>(sm, need);
      prefix |= sm.misc[0] << 10;
      need -= sm.misc[1];
      hist_begin<1024>(sm);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if ((mm[j >> 5] >> (j & 31)) & 1u) {
          const uint32_t k = order_key(v[j]);
          if ((k >> 10) == (prefix >> 10)) atomicAdd(&sm.hist[k & 1023u], 1u);
        }
      hist_end<1024>(sm, need);
      prefix |= sm.misc[0];
      const float thr = from_order_key(prefix);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (v[j] < thr) v[j] = -INFINITY;
    } else {
      mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NJ; ++j) mx = fmaxf(mx, v[j]);
      mx = block_max(mx, sm);
    }
    // From here v holds e = exp(y - max) of the filtered logits y (0 for the
    // removed ones), proportional to the probabilities p = e / S. Top-p keeps
    // the largest probability, so the maximum of what it leaves is the same,
    // and the distribution sample_from_logits draws from is e / (kept sum):
    // top-p zeroes entries in place.
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = v[j] > -INFINITY ? expf(v[j] - mx) : 0.f;
    float S = seg_total<NJ>(v, sm, w, lane);
    // ---- top-p (gpt2.rs:939-970): keep the largest probabilities, ties in
    // index order, until their running sum reaches p ----
    if (sp.top_p < 1.0f && sp.top_p > 0.0f) {
      // radix descent over the bits of e (non-negative floats order like their
      // bits), 10 + 11 + 10 bits, for the cut-off value with
      // mass(e > cut) < top_p <= mass(e >= cut); masses are summed as
      // integers (p * 2^31 rounded to nearest, mass_of): the same total in
      // any order
      const float ms = 2147483648.0f / S;  // 2^31 / S
      const unsigned target = max(1u, (unsigned)(sp.top_p * 2147483648.0f));
      hist_begin<1024>(sm);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (v[j] > 0.f) atomicAdd(&sm.hist[__float_as_uint(v[j]) >> 21], mass_of(v[j], ms));
      hist_end<1024>(sm, target);
      const uint32_t b1 = sm.misc[0];
      if (b1 != NONE) {  // else the total stays below p: everything is kept
        unsigned above = sm.misc[1];
        hist_begin<2048>(sm);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t k = __float_as_uint(v[j]);
          if (k != 0u && (k >> 21) == b1) atomicAdd(&sm.hist[(k >> 10) & 2047u], mass_of(v[j], ms));
        }
        hist_end<2048>(sm, target - above);
        const uint32_t p21 = (b1 << 11) | sm.misc[0];
        above += sm.misc[1];
        hist_begin<1024>(sm);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint32_t k = __float_as_uint(v[j]);
          if (k != 0u && (k >> 10) == p21) atomicAdd(&sm.hist[k & 1023u], mass_of(v[j], ms));
        }
        hist_end<1024>(sm, target - above);
        const uint32_t cut = (p21 << 10) | sm.misc[0];
        above += sm.misc[1];
        const unsigned qcut = mass_of(__uint_as_float(cut), ms);
        // entries equal to the cut-off all weigh qcut; the first `take` of them
        // in index order are kept, as many as the running sum needs to reach p
        const unsigned take = qcut ? (target - above + qcut - 1) / qcut : 0xffffffffu;
        const unsigned ties = qcut ? sm.misc[2] / qcut : 0xffffffffu;
        if (qcut == 0u || ties <= take) {
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            if (__float_as_uint(v[j]) < cut) v[j] = 0.f;
        } else {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const unsigned long long bal = __ballot(__float_as_uint(v[j]) == cut);
            if (lane == 0) sm.seg[j * SW + w] = (float)__popcll(bal);
          }
          __syncthreads();
          if (w == 0) wave_excl_prefix(sm.seg, sm.segpre, NJ * SW, lane);
          __syncthreads();
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const uint32_t k = __float_as_uint(v[j]);
            const bool tie = k == cut;
            const unsigned long long bal = __ballot(tie);
            bool keep = k > cut;
            if (tie) keep = (unsigned)sm.segpre[j * SW + w] + (unsigned)lanes_before(bal) < take;
            if (!keep) v[j] = 0.f;
          }
        }
        S = seg_total<NJ>(v, sm, w, lane);
      }
    }
    // ---- sample_from_logits (gpt2.rs:973-993): the first index whose
    // running sum of probabilities exceeds the uniform draw, here the first
    // whose running sum of e exceeds draw * S ----
    const float r = (float)(splitmix_at(sp.seed, (uint64_t)sp.draw0 + (uint64_t)g + 1) >> 40) * (1.0f / 16777216.0f);
    const float rs = r * S;
    if (w == 0) {
      // the (row, wave) segment of 64 indices where the running sum first exceeds rs
      const int n = NJ * SW;
      const int per = (n + 63) / 64, b0 = lane * per, e0 = min(n, b0 + per);
      int found = -1;
      for (int i = b0; i < e0 && found < 0; ++i)
        if (rs < sm.segpre[i] + sm.seg[i]) found = i;
      const unsigned long long bal = __ballot(found >= 0);
      const int segi = bal ? __shfl(found, __builtin_ctzll(bal), 64) : -1;
      if (lane == 0) {
        sm.misc[3] = segi < 0 ? NONE : (unsigned)segi;
        sm.fmisc[0] = segi < 0 ? 0.f : sm.segpre[segi];
      }
    }
    __syncthreads();
    const unsigned seg = sm.misc[3];
    if (seg == NONE) {
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
        const unsigned long long bal = __ballot(i < V && rs < sm.fmisc[0] + incl);
        // the segment's sum (a tree) put rs inside it; should the running sum
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

bool launch_sample(hipStream_t s, const float* logits, int V, const uint32_t* prompt, int n_prompt, uint32_t* ids,
                   const int* step_dev, const SampleParams& sp, uint32_t* token) {
#define RTG_SAMPLE(NJ) sample_kernel<NJ><<<1, ST, 0, s>>>(logits, V, prompt, n_prompt, ids, step_dev, sp, token)
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
