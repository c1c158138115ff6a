// Device side of the multi-row forward: forward_cached over a few rows (a
// short prompt of one sequence, or one new token of each of several
// sequences; rusttorch-core/src/nn/gpt2.rs:358-399, 477-538) in ONE launch on
// all 256 CUs, instead of ~11 kernels per layer.
//
// Rows: M = S * T <= 32, row r = sequence r / T, token r % T at position
// past + r % T. Every GEMM of a layer is cut into tiles of 32 output columns
// by a k range; tile i runs on workgroup i, whose four compute waves split
// the k range over the 32 (zero-padded) rows on fp32 MFMA (32x32x2). Tiles
// write partial sums; whoever consumes a GEMM's output adds them up in k
// order:
//   QKV    (c_attn on the LN1 output)  -> partials P0, summed + bias by ATT
//   ATT    items (sequence, head, group of 4 queries): q/k/v, the group's
//          k/v rows into the cache, causal attention over the cache (its
//          64-key blocks split between the four waves, each block scored
//          against all the group's queries) and the new rows (one query per
//          wave) -> O
//   PROJ   (attn c_proj on O)          -> partials P1
//   ROW2   one workgroup per row: x += P1 sums + bias; LN2(x) -> XN
//   FC     (c_fc on XN)                -> partials P0
//   MLP    (mlp c_proj on gelu_new(P0 sums + bias), formed as its operand
//          is read)                    -> partials P1
//   ROW3   x += P1 sums + bias; LN1 of the next layer (ln_f after the last)
//          -> XN
//   LM     tied LM head, every workgroup a strided set of 32-column tiles;
//          or, when the launch also takes the argmax for generate (at most
//          4 sequences), a GEMV over the last row of each sequence only.
// The residual row x stays in registers of its row workgroup for the whole
// forward. A fifth wave per workgroup only polls, so that the compute waves
// keep their weight prefetches (c_attn + attn c_proj at the start of a
// layer, c_fc + mlp c_proj at the start of the MLP half) in flight while the
// workgroup waits for its inputs. Nothing that does not depend on a wait is
// loaded after it (biases, LayerNorm rows): every load after a wait is one
// more memory round trip on the layer's critical path.
//
// Synchronisation: each workgroup owns one flag (a 64-bit word on its own
// 128-byte line) holding (epoch << 16) | sequence number of the last phase it
// finished. A producer's outputs are written with device-scope (sc1) stores
// on lines no other producer writes, its waves wait for them to complete,
// then one lane stores the flag; a consumer's poller wave polls the flags of
// exactly the producers it reads (device-scope loads). The epoch advances
// once per launch (by the last workgroup to finish), so flags never need
// clearing. Every wait is bounded: a timeout sets *err, later waits return at
// once, the launch finishes with wrong numbers and the host reports an error.
//
// Reads of data many workgroups share (the LayerNorm outputs, the attention
// output, the c_attn and c_fc partials), in FRESH mode: every (layer, phase)
// has its own region, written once per launch, so a plain load cannot meet a
// stale cached copy (caches are invalidated between launches) and the readers
// on one XCD share its L2. Device-scope loads of one shared region each (the
// mode of a caller-provided workspace too small for the layered regions)
// were measured 3-13 us per phase at 72-256 readers. Weight slices and (up to
// d = 768) the activation rows of a GEMM tile arrive by DMA into LDS as whole
// row runs (a lane-per-row load touches 64 lines per instruction: the MLP
// projection's input took 4.6 us that way); the MLP projection's weights,
// prefetched a phase ahead, come into registers. The MLP partials P1
// have one reader per row and are always read with device-scope loads from
// one region; every reuse of a region is ordered behind all of its readers
// through the flag graph (each reader is an ancestor of the next writer).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "argmax_key.h"
#include "attn_core.h"
#include "gelu.h"

namespace rtg {
namespace rk {

typedef unsigned long long u64;
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int G = 256;              // workgroups: one per CU of an MI355X
constexpr int NCW = 4;              // compute waves, one per SIMD
constexpr int NTH = 64 * (NCW + 1); // + the poller wave
constexpr int MR = 32;              // rows of every tile (MFMA 32x32)
constexpr int TN = 32;              // output columns of a GEMM tile
constexpr int HD = 64;              // head_dim
constexpr int TMAX = 32;            // new tokens per sequence
constexpr int SMAX = 16;            // sequences
constexpr int QG = 4;               // queries per attention item (one per compute wave)
constexpr int FS = 16;              // u64 words per flag slot (one 128-byte line)
constexpr int KWMAX = 64;           // k values per lane of a layer tile
constexpr int TRACE_WORDS = 1024;   // per workgroup: 4 per (layer, phase), t0 last
constexpr unsigned SPIN_CAP = 1u << 20;

// Phases of a layer in program order: a workgroup's flag only ever grows, so
// a flag at or past a phase's number means that phase's work is published.
enum { PH_QKV = 0, PH_ATT = 1, PH_PROJ = 2, PH_ROW2 = 3, PH_FC = 4, PH_MLP = 5, PH_ROW3 = 6 };
// Sequence number of phase ph of layer l; the embedding is PH_ROW3 of layer -1.
__host__ __device__ constexpr unsigned seq_of(int l, int ph) { return (unsigned)((l + 1) * 8 + ph); }

// k splits of a GEMM with ncols 32-column tiles over K: the largest split into
// whole 32-wide k ranges that keeps the tiles within one per workgroup and a
// lane's k values within KWMAX.
__host__ __device__ constexpr int pick_ks(int ncols, int K) {
  int best = 0;
  for (int ks = 1; ks * 32 <= K; ++ks)
    if (K % (32 * ks) == 0 && ncols * ks <= G && K / ks / 8 <= KWMAX) best = ks;
  return best;
}

template <int D>
struct RCfg {
  static constexpr int H = D / HD;
  static constexpr int NCQ = 3 * D / TN, KSQ = pick_ks(NCQ, D), KWQ = KSQ ? D / KSQ / 8 : 0, NTQ = NCQ * KSQ;
  static constexpr int NCP = D / TN, KSP = pick_ks(NCP, D), KWP = KSP ? D / KSP / 8 : 0, NTP = NCP * KSP;
  static constexpr int NCF = 4 * D / TN, KSF = pick_ks(NCF, D), KWF = KSF ? D / KSF / 8 : 0, NTF = NCF * KSF;
  static constexpr int NCM = D / TN, KSM = pick_ks(NCM, 4 * D), KWM = KSM ? 4 * D / KSM / 8 : 0,
                       NTM = NCM * KSM;
  static constexpr int NU = (D + 255) / 256;  // 16-byte chunks per lane of one row
  // floats of one layer's c_attn partials and c_fc partials, and of P1
  static constexpr long P0Q = (long)KSQ * MR * 3 * D, P0F = (long)KSF * MR * 4 * D;
  static constexpr long P1 = (long)(KSP > KSM ? KSP : KSM) * MR * D;
  static_assert(D % 64 == 0 && KSQ && KSP && KSF && KSM, "unsupported width");
  static_assert(KWQ % 4 == 0 && KWP % 4 == 0 && KWF % 4 == 0 && KWM % 4 == 0 && D % 128 == 0, "k chunks");
  static_assert(H * SMAX <= G, "attention items");
};

struct RLayer {
  const float *wqkv, *wproj, *wfc, *wmlp;  // W^T [N][K]
  const float *bqkv, *bproj, *bfc, *bmlp;
  const float *ln1w, *ln1b, *ln2w, *ln2b;
};

struct RParams {
  const RLayer* layers;
  const float *wte, *wpe, *lnfw, *lnfb;
  int L, P, V;
  float eps;
  float *kc, *vc;  // KV cache of layer 0 ([seq][head][P][64]); layer l at + l * kv_layer
  long kv_layer;
  int M, S, T;
  int past;            // position of every sequence's first new token ...
  const int* pos_dev;  // ... or, when set, *pos_dev
  const uint32_t* ids; // [M]
  // Regions (see the header comment); the strides are 0 outside FRESH mode.
  float* xn;  long xn_stride;  // LayerNorm outputs [MR][D]: 2l LN1 of layer l, 2l + 1 LN2, 2L ln_f
  float* o;   long o_stride;   // attention output [MR][D] of layer l
  float* p0;  long p0_stride;  // c_attn partials [KSQ][MR][3D] of layer l, then its c_fc partials
  long p0_fc;                  //   [KSF][MR][4D] at this offset
  float* p1;                   // attn / mlp c_proj partials [ks][MR][D]
  float* logits;       // [M][V]
  // Optional greedy finish (keys set): the argmax of each sequence's last row
  // (argmax_key, gpt2.rs:858-868) into keys[s]; the last workgroup to finish
  // then writes token[s] = that index and ids_out[s * ld_ids + *step], clears
  // the keys and advances *fin_pos and *step by one (the finalize of the
  // reference's generate loop, gpt2.rs:431-437).
  unsigned long long* keys;
  int lm_last;  // set (with keys, S <= LM_LAST_MAX): the LM head computes only each sequence's last row
  uint32_t* token;
  uint32_t* ids_out;
  int ld_ids;
  int* fin_pos;
  int* step;
  u64* flags;          // [G][FS]
  u64* epoch;
  unsigned* done;
  unsigned* err;
  u64* trace;          // optional: [G][TRACE_WORDS] phase timestamps
  // Test hook: the waits with code force_wait (0: none) wait for a flag
  // value no producer writes, so they time out after their SPIN_CAP polling
  // rounds (the error path, exercised without a fault or hang).
  unsigned force_wait;
};

#define RK_G(T, p) ((const __attribute__((address_space(1))) T*)(p))
#define RK_GW(T, p) ((__attribute__((address_space(1))) T*)(p))

// ---------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ u64 ld_flag(u64* f) {
  return __hip_atomic_load(RK_GW(u64, f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-scope 16-byte load of data written in this launch.
__device__ __forceinline__ float4 ldc4(const float* p) {
  u64* q = reinterpret_cast<u64*>(const_cast<float*>(p));
  const u64 a = __hip_atomic_load(RK_GW(u64, q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const u64 b = __hip_atomic_load(RK_GW(u64, q + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((unsigned)a), __uint_as_float((unsigned)(a >> 32)), __uint_as_float((unsigned)b),
                     __uint_as_float((unsigned)(b >> 32)));
}
__device__ __forceinline__ float4 ld4(const float* p) {
  const f4v v = *RK_G(f4v, p);
  return make_float4(v[0], v[1], v[2], v[3]);
}
// Load of data this launch wrote into a region of its own (FRESH) or into a
// shared region (device scope).
template <bool FRESH>
__device__ __forceinline__ float4 ldx4(const float* p) {
  if constexpr (FRESH) return ld4(p);
  else return ldc4(p);
}
template <bool FRESH>
__device__ __forceinline__ float ldx1(const float* p) {
  if constexpr (FRESH) return *RK_G(float, p);
  else return __hip_atomic_load(RK_GW(float, const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
  __hip_atomic_store(RK_GW(float, p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc4(float* p, float4 v) {
  u64* q = reinterpret_cast<u64*>(p);
  const u64 a = (u64)__float_as_uint(v.x) | ((u64)__float_as_uint(v.y) << 32);
  const u64 b = (u64)__float_as_uint(v.z) | ((u64)__float_as_uint(v.w) << 32);
  __hip_atomic_store(RK_GW(u64, q), a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(RK_GW(u64, q + 1), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 ldnt4(const float* p) {
  const f4v v = __builtin_nontemporal_load(RK_G(f4v, p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ bool err_set(const RParams& p) {
  return __hip_atomic_load(RK_GW(unsigned, p.err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ float wsum(float v) { return xor32_sum_k(xor16_sum_k(row16_sum_k(v))); }
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ u64 now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// The poller wave polls the flags of the n producers prod(0..n-1) until each
// holds at least target (bounded; a timeout sets *err with code); then the
// workgroup barrier releases the compute waves, whose weight loads stay in
// flight meanwhile.
template <class F>
__device__ __forceinline__ void wait_for(const RParams& p, int n, F prod, u64 target, unsigned code) {
  if (code == p.force_wait) target = ~0ull;
  if (wave_id() == NCW) {
    const int lane = threadIdx.x & 63;
    unsigned spins = 0;
    while (true) {
      // all of a lane's flags in flight at once (no short-circuit between them)
      // (branch-free: lanes past n re-read producer n - 1), as many rounds
      // of 64 as n needs
      u64 f[4];
      const int nr = (n + 63) >> 6;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < nr) f[k] = ld_flag(p.flags + (size_t)prod(min(lane + 64 * k, n - 1)) * FS);
      const bool failed = err_set(p);  // in the same round trip as the flags
      bool ok = true;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (k < nr) ok &= f[k] >= target;
      if (__all(ok)) break;
      if (++spins > SPIN_CAP || failed) {
        if (lane == 0 && spins > SPIN_CAP)
          __hip_atomic_store(RK_GW(unsigned, p.err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// Every wave's stores have completed; then one lane publishes the flag.
__device__ __forceinline__ void signal(const RParams& p, u64 val) {
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_store(RK_GW(u64, p.flags + (size_t)blockIdx.x * FS), val, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// GEMM tiles (compute waves)
// ---------------------------------------------------------------------------
// Lane (h = lane / 32, i = lane % 32) of compute wave w holds the k values
// kl + j (j < KW) of a tile's k range, kl = k0 + (2w + h) KW: W row n0 + i in
// w[], A row i in a[]. MFMA step j multiplies A[., kl + j] (lanes of half h
// supply k index h of the 32x32x2 block) with W[n0 + ., kl + j].

// 16 bytes per lane from global memory straight into LDS (64 lanes = 1 KiB
// at dst, lane i at dst + 16 i), streaming (nt). The loads count in vmcnt but
// occupy no registers; the compiler does not see them, so the wave waits for
// them itself (lds_dma_wait) before reading dst.
// POL: 0 streaming (nt: weights, read once), 1 cached (data in a region of
// its own), 2 device scope (data in a shared region).
template <int POL = 0>
__device__ __forceinline__ void lds_dma16(const float* src, float* dst) {
  const unsigned m0v =
      __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const __attribute__((address_space(3))) float*)dst);
  if constexpr (POL == 0)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(m0v) : "memory", "m0");
  else if constexpr (POL == 1)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0v) : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(src), "s"(m0v) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int LM_RING = 6;  // LM head weight slices in flight per wave (4 KiB each)
constexpr int LM_LAST_MAX = 4;  // sequences of the last-row LM head
// Waits until at most 4 n of this wave's memory instructions are outstanding
// (n = later LM head slices in flight, 4 DMA instructions each).
__device__ __forceinline__ void lm_wait(int n) {
  static_assert(LM_RING == 6, "one case per outstanding count");
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
  }
}

// LDS layout of a wave's weight slice: 32 rows (output columns n0 + i) x CPR
// 16-byte chunks (the wave's k range, both halves), chunk c of row i at slot
// i CPR + (c ^ swz(i)). The XOR spreads the 16 rows a quarter-wave reads over
// distinct banks; it stays inside the row because CPR is a multiple of 16
// (or 8) where it is applied.
template <int CPR>
__device__ __forceinline__ int swz(int row) {
  if constexpr (CPR % 16 == 0) return row & 15;
  else if constexpr (CPR % 8 == 0) return (row >> 1) & 7;
  else return 0;
}

// The wave's slice of a tile, W rows n0.. n0 + 31 (clamped to N - 1) over
// k [kw0, kw0 + 2 KW), into its LDS region wl (KW / 4 KiB): instruction t
// loads slots 64 t .. 64 t + 63, so each row's k range arrives as whole
// contiguous runs (in a permuted lane order).
template <int KW, int POL = 0>
__device__ __forceinline__ void w_dma(float* wl, const float* W, int K, int N, int n0, int kw0, int lane) {
  constexpr int CPR = KW / 2;
#pragma unroll
  for (int t = 0; t < KW / 4; ++t) {
    const int sl = 64 * t + lane, row = sl / CPR, c = (sl % CPR) ^ swz<CPR>(row);
    lds_dma16<POL>(W + (size_t)min(n0 + row, N - 1) * K + kw0 + 4 * c, wl + 256 * t);
  }
}
// The same for an activation slice: rows 0.. 31 of X (row stride ldx; rows
// past M re-read row M - 1: they only feed output rows that are never stored).
template <int KW, bool FRESH>
__device__ __forceinline__ void a_dma(float* al, const float* X, int ldx, int M, int kw0, int lane) {
  w_dma<KW, FRESH ? 1 : 2>(al, X, ldx, M, 0, kw0, lane);
}

template <int KW, bool FRESH>
__device__ __forceinline__ void a_rows(float4 (&a)[KW / 4], const float* X, int ldx, int M, int kl, int lane) {
  const int i = lane & 31;
  if (i < M) {
    const float* src = X + (size_t)i * ldx + kl;
#pragma unroll
    for (int j = 0; j < KW / 4; ++j) a[j] = ldx4<FRESH>(src + 4 * j);
  } else {
#pragma unroll
    for (int j = 0; j < KW / 4; ++j) a[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// MLP projection input in registers: gelu_new(c_fc partials summed in k
// order + bias), lane-per-row loads.
template <int KW, int KS, bool FRESH>
__device__ __forceinline__ void a_gelu(float4 (&a)[KW / 4], const float* P, int N, int M, const float* bias, int kl,
                                       int lane) {
  const int i = lane & 31;
  if (i < M) {
    float4 t[KS][KW / 4];
#pragma unroll
    for (int z = 0; z < KS; ++z)
#pragma unroll
      for (int j = 0; j < KW / 4; ++j) t[z][j] = ldx4<FRESH>(P + ((size_t)z * MR + i) * N + kl + 4 * j);
#pragma unroll
    for (int j = 0; j < KW / 4; ++j) {
      float4 s = t[0][j];
#pragma unroll
      for (int z = 1; z < KS; ++z) s = add4(s, t[z][j]);
      const float4 b = ld4(bias + kl + 4 * j);
      a[j] = make_float4(gelu_new(s.x + b.x), gelu_new(s.y + b.y), gelu_new(s.z + b.z), gelu_new(s.w + b.w));
    }
  } else {
#pragma unroll
    for (int j = 0; j < KW / 4; ++j) a[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// The wave's W values of a tile in registers, lane (h, i) = W[n0 + i][kl + 4j
// .. +4) (cached loads: the lines of 64 rows per instruction are re-read by
// the next ones from L2).
template <int KW>
__device__ __forceinline__ void w_regs(float4 (&w)[KW / 4], const float* W, int K, int N, int n0, int kl, int lane) {
  const float* src = W + (size_t)min(n0 + (lane & 31), N - 1) * K + kl;
#pragma unroll
  for (int j = 0; j < KW / 4; ++j) w[j] = ld4(src + 4 * j);
}

__device__ __forceinline__ void mma4(const float4& a, const float4& w, floatx16& c0, floatx16& c1) {
  c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, w.x, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, w.y, c1, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, w.z, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, w.w, c1, 0, 0, 0);
}

// W chunk q (k values kw0 + h KW + 4q ..) of lane (h, i) in w_dma's layout.
template <int KW>
__device__ __forceinline__ float4 w_chunk(const float* wl, int q, int lane) {
  constexpr int CPR = KW / 2;
  const int i = lane & 31, c = (lane >> 5) * (KW / 4) + q;
  return *reinterpret_cast<const float4*>(wl + 4 * (i * CPR + (c ^ swz<CPR>(i))));
}

// A and W from the wave's LDS regions (w_dma's layout).
template <int KW>
__device__ __forceinline__ floatx16 mma_lds(const float* al, const float* wl, int lane) {
  lds_dma_wait();
  floatx16 c0, c1;
#pragma unroll
  for (int e = 0; e < 16; ++e) c0[e] = c1[e] = 0.f;
#pragma unroll
  for (int j = 0; j < KW / 4; ++j) mma4(w_chunk<KW>(al, j, lane), w_chunk<KW>(wl, j, lane), c0, c1);
  return c0 + c1;
}

// A in registers, W from the wave's LDS region (w_dma's layout).
template <int KW>
__device__ __forceinline__ floatx16 mma_tile(const float4 (&a)[KW / 4], const float* wl, int lane) {
  lds_dma_wait();
  floatx16 c0, c1;
#pragma unroll
  for (int e = 0; e < 16; ++e) c0[e] = c1[e] = 0.f;
#pragma unroll
  for (int j = 0; j < KW / 4; ++j) mma4(a[j], w_chunk<KW>(wl, j, lane), c0, c1);
  return c0 + c1;
}

// Sums the compute waves' 32x32 tiles in wave order and hands element (row,
// column within the tile) to out(row, col, value): thread (q = tid / 64, l)
// gets rows 8q + 4 (l / 32) + u (u < 4) of column l % 32. Every wave passes
// both barriers.
template <class F>
__device__ __forceinline__ void tile_out(const floatx16& acc, float* red, int lane, F out) {
  const int wave = wave_id();
  if (wave < NCW) {
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(wave * 16 + e) * 64 + lane] = acc[e];
  }
  __syncthreads();
  if (wave < NCW) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = 4 * wave + u;
      float v = red[e * 64 + lane] + red[(16 + e) * 64 + lane];
      v += red[(32 + e) * 64 + lane];
      v += red[(48 + e) * 64 + lane];
      out(8 * wave + 4 * (lane >> 5) + u, lane & 31, v);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// rows: residual add of a GEMM's partials and the LayerNorm after it
// ---------------------------------------------------------------------------

// A row's NU 16-byte chunks of v (lane's chunks lane + 64 u, clamped).
template <int D>
__device__ __forceinline__ void row_load(float4 (&r)[RCfg<D>::NU], const float* v, int lane) {
#pragma unroll
  for (int u = 0; u < RCfg<D>::NU; ++u) r[u] = ld4(v + 4 * min(lane + 64 * u, D / 4 - 1));
}

// LayerNorm of the row in x (gpt2.rs:636-666: mean, then the mean of squared
// deviations, (x - mean) / sqrt(var + eps) * g + b) into row xn_row; gv, bv:
// the gain and bias chunks (row_load), loaded ahead.
template <int D>
__device__ __forceinline__ void row_ln(const float4 (&x)[RCfg<D>::NU], const float4 (&gv)[RCfg<D>::NU],
                                       const float4 (&bv)[RCfg<D>::NU], float eps, float* xn_row, int lane) {
  constexpr int NU = RCfg<D>::NU, NC = D / 4;
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u)
    if (lane + 64 * u < NC) sum += (x[u].x + x[u].y) + (x[u].z + x[u].w);
  const float mean = wsum(sum) / (float)D;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u)
    if (lane + 64 * u < NC) {
      const float a = x[u].x - mean, bb = x[u].y - mean, c = x[u].z - mean, d = x[u].w - mean;
      sq += (a * a + bb * bb) + (c * c + d * d);
    }
  const float var = wsum(sq) / (float)D;
  const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int ch = lane + 64 * u;
    if (ch < NC)
      stc4(xn_row + 4 * ch, make_float4((x[u].x - mean) * inv_std * gv[u].x + bv[u].x,
                                        (x[u].y - mean) * inv_std * gv[u].y + bv[u].y,
                                        (x[u].z - mean) * inv_std * gv[u].z + bv[u].z,
                                        (x[u].w - mean) * inv_std * gv[u].w + bv[u].w));
  }
}

// x += (sum of the KS partial rows in k order) + bias (gpt2.rs:517-537: the
// residual add of the projection's output, bias included; bias: row_load's
// chunks, loaded ahead).
template <int D, int KS>
__device__ __forceinline__ void row_resid(float4 (&x)[RCfg<D>::NU], const float* P, int r,
                                          const float4 (&bias)[RCfg<D>::NU], int lane) {
  constexpr int NU = RCfg<D>::NU, NC = D / 4;
  float4 t[KS][NU];
#pragma unroll
  for (int z = 0; z < KS; ++z)
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int ch = min(lane + 64 * u, NC - 1);
      t[z][u] = ldc4(P + ((size_t)z * MR + r) * D + 4 * ch);
    }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int ch = lane + 64 * u;
    if (ch < NC) {
      float4 s = t[0][u];
#pragma unroll
      for (int z = 1; z < KS; ++z) s = add4(s, t[z][u]);
      const float4 b = bias[u];
      x[u] = add4(x[u], make_float4(s.x + b.x, s.y + b.y, s.z + b.z, s.w + b.w));
    }
  }
}

// ---------------------------------------------------------------------------
// attention items (multi_head_attention_cached, gpt2.rs:772-834): item =
// (sequence s, head h, query group g): queries t in [g QG, g QG + QG) of the T
// new rows, one per compute wave
// ---------------------------------------------------------------------------

struct AttLds {
  float q[TMAX * HD];
  float k[TMAX * (HD + 4)];  // padded rows: lane-per-key reads spread over the banks
  float v[TMAX * HD];
  float mg[NCW][QG][HD + 2];  // each wave's (o, m, l) per query, merged over the waves
};

// One block of up to 64 keys [kb, kb + nk) of query t, keys from the cache
// rows K / V (row stride HD, FROM_LDS false) or from the item's new rows in
// LDS (row key - past): online softmax update of (m, l, o), lane = key for the
// scores and lane = dim for the output.
template <bool FROM_LDS>
__device__ __forceinline__ void att_block(const AttLds& A, int t, int past, const float* K, const float* Vg, int kb,
                                          int nk, float& m, float& l, float& o, int lane) {
  const float scale = 0.125f;  // 1 / sqrt(64)
  const float4* q4 = reinterpret_cast<const float4*>(A.q + t * HD);
  const bool valid = lane < nk;
  float dot = 0.f;
  if (valid) {
    if constexpr (FROM_LDS) {
      const float4* kr = reinterpret_cast<const float4*>(A.k + (kb + lane - past) * (HD + 4));
#pragma unroll
      for (int c = 0; c < HD / 4; ++c) {
        const float4 kk = kr[c], qq = q4[c];
        dot += qq.x * kk.x + qq.y * kk.y + qq.z * kk.z + qq.w * kk.w;
      }
    } else {
      const float* kr = K + (size_t)(kb + lane) * HD;
#pragma unroll
      for (int c = 0; c < HD / 4; ++c) {
        const float4 kk = ld4(kr + 4 * c), qq = q4[c];
        dot += qq.x * kk.x + qq.y * kk.y + qq.z * kk.z + qq.w * kk.w;
      }
    }
  }
  const float sc = valid ? dot * scale : -__builtin_inff();
  const float mn = fmaxf(m, wmax(sc));
  const float pe = valid ? fexp_a(sc - mn) : 0.f;
  const float corr = fexp_a(m - mn);
  l = l * corr + wsum(pe);
  o *= corr;
  int i = 0;
  for (; i + 8 <= nk; i += 8) {
    float vv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if constexpr (FROM_LDS) vv[u] = A.v[(kb + i + u - past) * HD + lane];
      else vv[u] = Vg[(size_t)(kb + i + u) * HD + lane];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) o += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), i + u)) * vv[u];
  }
  for (; i < nk; ++i) {
    float vv;
    if constexpr (FROM_LDS) vv = A.v[(kb + i - past) * HD + lane];
    else vv = Vg[(size_t)(kb + i) * HD + lane];
    o += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe), i)) * vv;
  }
  m = mn;
}

// Cache keys [kb, kb + nk) (all below past, so every query sees them) against
// the nq queries t_lo .. of the item at once: lane = key for the scores, lane
// = dim for the outputs; the block's K and V rows are read once for all the
// queries.
__device__ __forceinline__ void att_cache_block(const AttLds& A, int t_lo, int nq, const float* K, const float* Vg,
                                                int kb, int nk, float (&m)[QG], float (&l)[QG], float (&o)[QG],
                                                int lane) {
  const bool valid = lane < nk;
  const float* kr = K + (size_t)(kb + min(lane, nk - 1)) * HD;
  float4 kv[HD / 4];
#pragma unroll
  for (int c = 0; c < HD / 4; ++c) kv[c] = ld4(kr + 4 * c);
  float pe[QG];
#pragma unroll
  for (int q = 0; q < QG; ++q) {
    pe[q] = 0.f;
    if (q < nq) {  // wave-uniform
      const float4* q4 = reinterpret_cast<const float4*>(A.q + (t_lo + q) * HD);
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < HD / 4; ++c) {
        const float4 qq = q4[c];
        dot += qq.x * kv[c].x + qq.y * kv[c].y + qq.z * kv[c].z + qq.w * kv[c].w;
      }
      const float sc = valid ? dot * 0.125f : -__builtin_inff();  // 1 / sqrt(64)
      const float mn = fmaxf(m[q], wmax(sc));
      pe[q] = valid ? fexp_a(sc - mn) : 0.f;
      const float corr = fexp_a(m[q] - mn);
      l[q] = l[q] * corr + wsum(pe[q]);
      o[q] *= corr;
      m[q] = mn;
    }
  }
  for (int i = 0; i < nk; i += 8) {
    float vv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) vv[u] = Vg[(size_t)(kb + min(i + u, nk - 1)) * HD + lane];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (i + u < nk) {  // wave-uniform
#pragma unroll
        for (int q = 0; q < QG; ++q)
          if (q < nq) o[q] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pe[q]), i + u)) * vv[u];
      }
    }
  }
}

// Keys [0, k_hi) of query t in blocks of 64 (b0, b0 + bstep, ...): the cache
// rows below past, then the new rows.
__device__ __forceinline__ void att_range(const AttLds& A, int t, int past, const float* Kc, const float* Vc,
                                          int k_hi, int b0, int bstep, float& m, float& l, float& o, int lane) {
  const int nb_c = (past + 63) / 64;              // blocks over the cache rows
  const int nb = nb_c + (k_hi - past + 63) / 64;  // then over the new rows
  for (int b = b0; b < nb; b += bstep) {
    if (b < nb_c) {
      const int kb = 64 * b;
      att_block<false>(A, t, past, Kc, Vc, kb, min(64, past - kb), m, l, o, lane);
    } else {
      const int kb = past + 64 * (b - nb_c);
      att_block<true>(A, t, past, Kc, Vc, kb, min(64, k_hi - kb), m, l, o, lane);
    }
  }
}

// q of the group's queries and k / v of rows [0, t_hi): the c_attn partials
// summed in k order, + bias, into LDS; the group's own k / v rows also into
// the cache at past + t. All of a thread's partial loads are in flight
// together. Compute waves only; the caller's barrier follows.
template <int D, bool FRESH>
__device__ __forceinline__ void att_gather(const RParams& p, AttLds& A, const float* P0, int l, int s, int h,
                                           int t_lo, int t_hi, int past, float* Kc, float* Vc, int tid) {
  constexpr int KS = RCfg<D>::KSQ, NCT = NCW * 64;
  constexpr int EMAX = (QG * (HD / 4) + 2 * TMAX * (HD / 4) + NCT - 1) / NCT;
  const int T = p.T;
  const int nq = (t_hi - t_lo) * (HD / 4), nkv = t_hi * (HD / 4);
  const int n4 = nq + 2 * nkv;
  const float* bq = p.layers[l].bqkv;
  auto decode = [&](int e, int& part, int& t, int& d4) {
    if (e < nq) {
      part = 0;
      t = t_lo + e / (HD / 4);
      d4 = e % (HD / 4);
    } else {
      const int f = e - nq;
      part = 1 + f / nkv;
      t = (f % nkv) / (HD / 4);
      d4 = f % (HD / 4);
    }
  };
  float4 v[EMAX][KS], bb[EMAX];
#pragma unroll
  for (int i = 0; i < EMAX; ++i) {
    const int e = tid + NCT * i;
    if (e < n4) {
      int part, t, d4;
      decode(e, part, t, d4);
      const int col = part * D + h * HD + 4 * d4, r = s * T + t;
#pragma unroll
      for (int z = 0; z < KS; ++z) v[i][z] = ldx4<FRESH>(P0 + ((size_t)z * MR + r) * (3 * D) + col);
      bb[i] = ld4(bq + col);  // with the partials, not a round trip after them
    }
  }
#pragma unroll
  for (int i = 0; i < EMAX; ++i) {
    const int e = tid + NCT * i;
    if (e < n4) {
      int part, t, d4;
      decode(e, part, t, d4);
      const int col = part * D + h * HD + 4 * d4;
      float4 sum = v[i][0];
#pragma unroll
      for (int z = 1; z < KS; ++z) sum = add4(sum, v[i][z]);
      const float4 b = bb[i];
      const float4 x = make_float4(sum.x + b.x, sum.y + b.y, sum.z + b.z, sum.w + b.w);
      if (part == 0) {
        *reinterpret_cast<float4*>(A.q + t * HD + 4 * d4) = x;
      } else if (part == 1) {
        *reinterpret_cast<float4*>(A.k + t * (HD + 4) + 4 * d4) = x;
        if (t >= t_lo) *reinterpret_cast<float4*>(Kc + (size_t)(past + t) * HD + 4 * d4) = x;
      } else {
        *reinterpret_cast<float4*>(A.v + t * HD + 4 * d4) = x;
        if (t >= t_lo) *reinterpret_cast<float4*>(Vc + (size_t)(past + t) * HD + 4 * d4) = x;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------

// LDS of a workgroup: more than half of the CU's 160 KiB (padded where the
// width leaves it smaller), so that no two workgroups share a CU.
template <int D>
struct RSmem {
  using C = RCfg<D>;
  // activation slices through LDS as well where it has room for them
  static constexpr bool ADMA = D <= 768;
  // per-wave slices (w_dma layout): the c_attn and attn c_proj weights in the
  // first half of a layer (c_attn's activations where the attention items'
  // LDS goes later; attn c_proj's where the c_attn weights were), the c_fc
  // weights and activations in the second, replaced by mlp c_proj's once c_fc
  // is computed
  static constexpr int WQ = NCW * C::KWQ * 64, WP = NCW * C::KWP * 64;
  static constexpr int WF = NCW * C::KWF * 64, WM = NCW * C::KWM * 64;
  // the second half: c_fc's weights and activations, then the KSF c_fc
  // partial slices of the mlp c_proj's input
  static constexpr int H2A = 2 * WF, H2B = C::KSF * WM + NCW * 256;  // + each wave's c_fc bias slice
  static constexpr int H2 = ADMA ? (H2A > H2B ? H2A : H2B) : WF;
  struct Half1 {
    float wq[WQ];
    float wp[WP];
    union {
      AttLds att;
      float aq[ADMA ? WQ : 1];
    };
  };
  struct Half2 {
    float x[H2];
  };
  float red[NCW * 16 * 64];  // the compute waves' 32x32 tiles
  u64 trs[TRACE_WORDS];
  union {
    Half1 h1;
    Half2 h2;
    float lmw[NCW * LM_RING * 1024];  // the LM head's per-wave weight rings
  };
  static constexpr int U1 = (int)sizeof(Half1), U2 = (int)sizeof(Half2), U3 = NCW * LM_RING * 1024 * 4;
  static constexpr int BASE = NCW * 16 * 64 * 4 + TRACE_WORDS * 8 + (U1 > U2 ? (U1 > U3 ? U1 : U3) : (U2 > U3 ? U2 : U3));
  float pad[BASE < 84 * 1024 ? (84 * 1024 - BASE) / 4 : 1];
};

template <int D, bool FRESH>
__global__ __launch_bounds__(NTH, 1) void rows_kernel(RParams p) {
  using C = RCfg<D>;
  constexpr int H = C::H, NU = C::NU;
  __shared__ RSmem<D> sm;
  static_assert(sizeof(RSmem<D>) <= 160 * 1024, "LDS");
  constexpr bool ADMA = RSmem<D>::ADMA;
  // row phases load their bias and LayerNorm rows before waiting (registers
  // allow it up to 768 wide; wider rows load them with the partials)
  constexpr bool RPF = D <= 768;
  static_assert(!ADMA || C::KWP <= C::KWQ, "attn c_proj activations in the c_attn weight region");
  float* red = sm.red;
  AttLds& att = sm.h1.att;
  u64* trs = sm.trs;
  const int wg = blockIdx.x, tid0 = threadIdx.x, wave = wave_id();
  const bool cw = wave < NCW;  // compute wave
  const u64 E = __hip_atomic_load(RK_GW(u64, p.epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) << 16;
  const int M = p.M, S = p.S, T = p.T, L = p.L;
  const int past = p.pos_dev ? *RK_G(int, p.pos_dev) : p.past;
  const int my_row = wg >= G - M ? G - 1 - wg : -1;
  const int ngr = (T + QG - 1) / QG;  // query groups per (sequence, head)
  const int my_item = G - 1 - wg < S * H * ngr ? G - 1 - wg : -1;
  const bool tracing = p.trace != nullptr && (L + 2) * 32 < TRACE_WORDS;
  if (tracing)
    for (int i = tid0; i < TRACE_WORDS; i += NTH) trs[i] = 0;
  const u64 t0 = now();
  // k: 0 inputs ready, 1 operands in / gathered, 2 computed, 3 published
  auto mark = [&](int l, int ph, int k) {
    if (tracing && tid0 == 0) trs[((l + 1) * 8 + ph) * 4 + k] = now() - t0;
  };
  // the same once v (a loaded or computed value) is available
  auto markv = [&](int l, int ph, int k, float v) {
    if (tracing) {
      asm volatile("" ::"v"(v));
      mark(l, ph, k);
    }
  };
  auto row_wg = [&](int i) { return G - 1 - i; };
  auto xn_of = [&](int inst) { return p.xn + inst * p.xn_stride; };
  float4 xr[NU];

  // ---- embedding (gpt2.rs:377-384) and LN1 of layer 0 ----
  if (my_row >= 0) {
    const int lane = tid0 & 63;
    if (wave == 0) {
      const uint32_t id = p.ids[my_row];
      const int pos = past + my_row % T;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int ch = min(lane + 64 * u, D / 4 - 1);
        xr[u] = add4(ld4(p.wte + (size_t)id * D + 4 * ch), ld4(p.wpe + (size_t)pos * D + 4 * ch));
      }
      float4 gv[NU], bv[NU];
      row_load<D>(gv, L ? p.layers[0].ln1w : p.lnfw, lane);
      row_load<D>(bv, L ? p.layers[0].ln1b : p.lnfb, lane);
      row_ln<D>(xr, gv, bv, p.eps, xn_of(0) + (size_t)my_row * D, lane);
    }
    signal(p, E | seq_of(-1, PH_ROW3));
    mark(-1, PH_ROW3, 3);
  }

  for (int l = 0; l < L; ++l) {
    // per-lane indices recomputed every layer from an opaque copy, so that the
    // compiler does not hoist every phase's lane addresses out of the loop
    // (they would not fit the registers beside the prefetched weights)
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const RLayer& Lw = p.layers[l];
    const float* xn1 = xn_of(2 * l);
    float* xn2 = xn_of(2 * l + 1);
    float* ol = p.o + l * p.o_stride;
    float* p0q = p.p0 + l * p.p0_stride;
    float* p0f = p0q + p.p0_fc;
    // weights of this layer's c_attn and attn c_proj tiles, in flight into LDS from here
    float* wq = sm.h1.wq + wave * C::KWQ * 64;
    float* wp = sm.h1.wp + wave * C::KWP * 64;
    // k range of this compute wave in its tile (kw0: both halves) and of this lane (kl)
    const int cq = wg / C::KSQ, zq = wg % C::KSQ;
    const int kwq = zq * (D / C::KSQ) + 2 * wave * C::KWQ, klq = kwq + (lane >> 5) * C::KWQ;
    const int cp = wg / C::KSP, zp = wg % C::KSP;
    constexpr int KCP = D / C::KSP;
    const int kwp = zp * KCP + 2 * wave * C::KWP, klp = kwp + (lane >> 5) * C::KWP;
    if (cw && wg < C::NTQ) w_dma<C::KWQ>(wq, Lw.wqkv, D, 3 * D, cq * TN, kwq, lane);
    if (cw && wg < C::NTP) w_dma<C::KWP>(wp, Lw.wproj, D, D, cp * TN, kwp, lane);

    // ---- c_attn (LN1 output) -> P0 ----
    if (wg < C::NTQ) {
      wait_for(p, M, row_wg, E | seq_of(l - 1, PH_ROW3), 1);
      mark(l, PH_QKV, 0);
      floatx16 acc = {};  // (the poller wave passes zeros to tile_out)
      if (cw) {
        if constexpr (ADMA) {
          float* aq = sm.h1.aq + wave * C::KWQ * 64;
          a_dma<C::KWQ, FRESH>(aq, xn1, D, M, kwq, lane);
          lds_dma_wait();
          mark(l, PH_QKV, 1);
          acc = mma_lds<C::KWQ>(aq, wq, lane);
        } else {
          float4 a[C::KWQ / 4];
          a_rows<C::KWQ, FRESH>(a, xn1, D, M, klq, lane);
          markv(l, PH_QKV, 1, a[C::KWQ / 4 - 1].w);
          acc = mma_tile<C::KWQ>(a, wq, lane);
        }
        markv(l, PH_QKV, 2, acc[15]);
      }
      const int n0 = cq * TN;
      tile_out(acc, red, lane, [&](int r, int cc, float v) {
        if (r < M) stc(p0q + ((size_t)zq * MR + r) * (3 * D) + n0 + cc, v);
      });
      signal(p, E | seq_of(l, PH_QKV));
      mark(l, PH_QKV, 3);
    }
    // ---- attention items ----
    if (my_item >= 0) {
      const int g = my_item % ngr, sh = my_item / ngr, s = sh / H, h = sh % H;
      const int t_lo = g * QG, t_hi = min(T, g * QG + QG);
      // the c_attn tiles of head h's q, k and v columns
      auto prod = [&](int i) {
        const int z = i % C::KSQ, j = i / C::KSQ;  // j < 6: part j / 2, column tile 2h + j % 2
        return ((j >> 1) * (D / TN) + 2 * h + (j & 1)) * C::KSQ + z;
      };
      wait_for(p, 6 * C::KSQ, prod, E | seq_of(l, PH_QKV), 2);
      mark(l, PH_ATT, 0);
      float* Kc = p.kc + l * p.kv_layer + (size_t)(s * H + h) * p.P * HD;
      float* Vc = p.vc + l * p.kv_layer + (size_t)(s * H + h) * p.P * HD;
      if (cw) att_gather<D, FRESH>(p, att, p0q, l, s, h, t_lo, t_hi, past, Kc, Vc, tid);
      __syncthreads();
      mark(l, PH_ATT, 1);
      if (past == 0 || D > 768) {
        // no cached rows (or the width whose registers cannot hold the
        // key-parallel form): wave w attends query t_lo + w over all its keys
        if (cw && t_lo + wave < t_hi) {
          const int t = t_lo + wave;
          float m = -__builtin_inff(), ll = 0.f, o = 0.f;
          att_range(att, t, past, Kc, Vc, past + t + 1, 0, 1, m, ll, o, lane);
          stc(ol + (size_t)(s * T + t) * D + h * HD + lane, o / ll);
        }
      } else {
        // cached rows: wave w takes the 64-key blocks w, w + 4, ... of the
        // cache for all the item's queries; wave q then adds query t_lo + q's
        // new rows; the waves' states merge in wave order
        const int nq = t_hi - t_lo;
        float m[QG], ll[QG], o[QG];
#pragma unroll
        for (int q = 0; q < QG; ++q) {
          m[q] = -__builtin_inff();
          ll[q] = 0.f;
          o[q] = 0.f;
        }
        if (cw) {
          for (int kb = 64 * wave; kb < past; kb += 64 * NCW)
            att_cache_block(att, t_lo, nq, Kc, Vc, kb, min(64, past - kb), m, ll, o, lane);
#pragma unroll
          for (int q = 0; q < QG; ++q)
            if (q == wave && q < nq)
              att_block<true>(att, t_lo + q, past, Kc, Vc, past, t_lo + q + 1, m[q], ll[q], o[q], lane);
#pragma unroll
          for (int q = 0; q < QG; ++q) {
            att.mg[wave][q][2 + lane] = o[q];
            if (lane == 0) {
              att.mg[wave][q][0] = m[q];
              att.mg[wave][q][1] = ll[q];
            }
          }
        }
        __syncthreads();
        if (cw && wave < nq) {
          const int q = wave;
          float M = -__builtin_inff();
#pragma unroll
          for (int w = 0; w < NCW; ++w) M = fmaxf(M, att.mg[w][q][0]);
          float L = 0.f, O = 0.f;
#pragma unroll
          for (int w = 0; w < NCW; ++w) {
            const float mw = att.mg[w][q][0];
            const float f = mw == -__builtin_inff() ? 0.f : fexp_a(mw - M);
            L += att.mg[w][q][1] * f;
            O += att.mg[w][q][2 + lane] * f;
          }
          stc(ol + (size_t)(s * T + t_lo + q) * D + h * HD + lane, O / L);
        }
      }
      mark(l, PH_ATT, 2);
      signal(p, E | seq_of(l, PH_ATT));
      mark(l, PH_ATT, 3);
    }
    // ---- attention c_proj (O) -> P1 ----
    if (wg < C::NTP) {
      // the attention items of the heads this k range covers, every sequence and query group
      const int h0 = zp * KCP / HD, nh = (zp * KCP + KCP - 1) / HD - h0 + 1;
      wait_for(
          p, nh * S * ngr,
          [&](int i) {
            const int g = i % ngr, j = i / ngr;
            return G - 1 - (((j / nh) * H + h0 + j % nh) * ngr + g);
          },
          E | seq_of(l, PH_ATT), 3);
      mark(l, PH_PROJ, 0);
      floatx16 acc = {};  // (the poller wave passes zeros to tile_out)
      if (cw) {
        if constexpr (ADMA) {
          float* ap = sm.h1.wq + wave * C::KWP * 64;  // the c_attn weights are consumed
          a_dma<C::KWP, FRESH>(ap, ol, D, M, kwp, lane);
          lds_dma_wait();
          mark(l, PH_PROJ, 1);
          acc = mma_lds<C::KWP>(ap, wp, lane);
        } else {
          float4 a[C::KWP / 4];
          a_rows<C::KWP, FRESH>(a, ol, D, M, klp, lane);
          markv(l, PH_PROJ, 1, a[C::KWP / 4 - 1].w);
          acc = mma_tile<C::KWP>(a, wp, lane);
        }
        markv(l, PH_PROJ, 2, acc[15]);
      }
      const int n0 = cp * TN;
      tile_out(acc, red, lane, [&](int r, int cc, float v) {
        if (r < M) stc(p.p1 + ((size_t)zp * MR + r) * D + n0 + cc, v);
      });
      signal(p, E | seq_of(l, PH_PROJ));
      mark(l, PH_PROJ, 3);
    }
    // ---- x += attention output; LN2 -> XN ----
    if (my_row >= 0) {
      // the bias, gain and LN bias rows: before the wait where the registers
      // allow (they do not depend on it), else with the partials
      float4 bv[NU], gv[NU], lv[NU];
      auto params = [&] {
        row_load<D>(bv, Lw.bproj, lane);
        row_load<D>(gv, Lw.ln2w, lane);
        row_load<D>(lv, Lw.ln2b, lane);
      };
      if (RPF && wave == 0) params();
      wait_for(p, C::NTP, [](int i) { return i; }, E | seq_of(l, PH_PROJ), 4);
      mark(l, PH_ROW2, 0);
      if (wave == 0) {
        if (!RPF) params();
        row_resid<D, C::KSP>(xr, p.p1, my_row, bv, lane);
        markv(l, PH_ROW2, 1, xr[0].x);
        row_ln<D>(xr, gv, lv, p.eps, xn2 + (size_t)my_row * D, lane);
      }
      signal(p, E | seq_of(l, PH_ROW2));
      mark(l, PH_ROW2, 3);
    }
    // c_fc weights (into LDS) in flight from here (after the row workgroups'
    // LayerNorm, whose registers they would otherwise share); mlp c_proj's
    // (into registers) once c_fc's stores are issued
    float* wf = sm.h2.x + wave * C::KWF * 64;
    const int cf = wg / C::KSF, zf = wg % C::KSF;
    const int kwf = zf * (D / C::KSF) + 2 * wave * C::KWF, klf = kwf + (lane >> 5) * C::KWF;
    const int cm = wg / C::KSM, zm = wg % C::KSM;
    constexpr int KCM = 4 * D / C::KSM;
    const int kwm = zm * KCM + 2 * wave * C::KWM, klm = kwm + (lane >> 5) * C::KWM;
    float4 wm[C::KWM / 4];
#pragma unroll
    for (int j = 0; j < C::KWM / 4; ++j) wm[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (cw && wg < C::NTF) w_dma<C::KWF>(wf, Lw.wfc, D, 4 * D, cf * TN, kwf, lane);
    // ---- c_fc (LN2 output) -> P0 ----
    if (wg < C::NTF) {
      // mlp c_proj's weights (registers) while the row phase runs: issued
      // after c_fc's, all 192 tiles' loads would meet c_fc's publication
      if (wg < C::NTM && cw) w_regs<C::KWM>(wm, Lw.wmlp, 4 * D, D, cm * TN, klm, lane);
      wait_for(p, M, row_wg, E | seq_of(l, PH_ROW2), 5);
      mark(l, PH_FC, 0);
      floatx16 acc = {};  // (the poller wave passes zeros to tile_out)
      if (cw) {
        if constexpr (ADMA) {
          float* af = sm.h2.x + RSmem<D>::WF + wave * C::KWF * 64;
          a_dma<C::KWF, FRESH>(af, xn2, D, M, kwf, lane);
          lds_dma_wait();
          mark(l, PH_FC, 1);
          acc = mma_lds<C::KWF>(af, wf, lane);
        } else {
          float4 a[C::KWF / 4];
          a_rows<C::KWF, FRESH>(a, xn2, D, M, klf, lane);
          markv(l, PH_FC, 1, a[C::KWF / 4 - 1].w);
          acc = mma_tile<C::KWF>(a, wf, lane);
        }
        markv(l, PH_FC, 2, acc[15]);
      }
      const int n0 = cf * TN;
      tile_out(acc, red, lane, [&](int r, int cc, float v) {
        if (r < M) stc(p0f + ((size_t)zf * MR + r) * (4 * D) + n0 + cc, v);
      });
      signal(p, E | seq_of(l, PH_FC));
      mark(l, PH_FC, 3);
    }
    // ---- mlp c_proj (gelu_new of the c_fc output) -> P1 ----
    if (wg < C::NTM) {
      if (cw && wg >= C::NTF) w_regs<C::KWM>(wm, Lw.wmlp, 4 * D, D, cm * TN, klm, lane);
      // the c_fc tiles of columns [zm KCM, zm KCM + KCM), every k split
      wait_for(
          p, (KCM / TN) * C::KSF, [&](int i) { return (zm * (KCM / TN) + i / C::KSF) * C::KSF + i % C::KSF; },
          E | seq_of(l, PH_FC), 6);
      mark(l, PH_MLP, 0);
      floatx16 acc = {};  // (the poller wave passes zeros to tile_out)
      if (cw) {
        if constexpr (ADMA) {
          // the KSF partial slices into LDS (where c_fc's weights and
          // activations were), summed in k order + bias, gelu_new, as read
          float* am = sm.h2.x + wave * C::KWM * 64;
#pragma unroll
          for (int z = 0; z < C::KSF; ++z)
            a_dma<C::KWM, FRESH>(am + z * RSmem<D>::WM, p0f + (size_t)z * MR * (4 * D), 4 * D, M, kwm, lane);
          // the bias of the wave's k range (2 KWM values; lanes past it re-read its last chunk)
          float* bl = sm.h2.x + C::KSF * RSmem<D>::WM + wave * 256;
          lds_dma16<1>(Lw.bfc + kwm + 4 * min(lane, C::KWM / 2 - 1), bl);
          lds_dma_wait();
          mark(l, PH_MLP, 1);
          floatx16 c0, c1;
#pragma unroll
          for (int e = 0; e < 16; ++e) c0[e] = c1[e] = 0.f;
#pragma unroll
          for (int j = 0; j < C::KWM / 4; ++j) {
            float4 t = w_chunk<C::KWM>(am, j, lane);
#pragma unroll
            for (int z = 1; z < C::KSF; ++z) t = add4(t, w_chunk<C::KWM>(am + z * RSmem<D>::WM, j, lane));
            const float4 b = *reinterpret_cast<const float4*>(bl + (lane >> 5) * C::KWM + 4 * j);
            const float4 av =
                make_float4(gelu_new(t.x + b.x), gelu_new(t.y + b.y), gelu_new(t.z + b.z), gelu_new(t.w + b.w));
            mma4(av, wm[j], c0, c1);
          }
          acc = c0 + c1;
        } else {
          float4 a[C::KWM / 4];
          a_gelu<C::KWM, C::KSF, FRESH>(a, p0f, 4 * D, M, Lw.bfc, klm, lane);
          markv(l, PH_MLP, 1, a[C::KWM / 4 - 1].w);
          floatx16 c0, c1;
#pragma unroll
          for (int e = 0; e < 16; ++e) c0[e] = c1[e] = 0.f;
#pragma unroll
          for (int j = 0; j < C::KWM / 4; ++j) mma4(a[j], wm[j], c0, c1);
          acc = c0 + c1;
        }
        markv(l, PH_MLP, 2, acc[15]);
      }
      const int n0 = cm * TN;
      tile_out(acc, red, lane, [&](int r, int cc, float v) {
        if (r < M) stc(p.p1 + ((size_t)zm * MR + r) * D + n0 + cc, v);
      });
      signal(p, E | seq_of(l, PH_MLP));
      mark(l, PH_MLP, 3);
    }
    // ---- x += MLP output; LN1 of the next layer (ln_f after the last) -> XN ----
    if (my_row >= 0) {
      const bool last = l + 1 == L;
      float4 bv[NU], gv[NU], lv[NU];
      auto params = [&] {
        row_load<D>(bv, Lw.bmlp, lane);
        row_load<D>(gv, last ? p.lnfw : p.layers[l + 1].ln1w, lane);
        row_load<D>(lv, last ? p.lnfb : p.layers[l + 1].ln1b, lane);
      };
      if (RPF && wave == 0) params();
      wait_for(p, C::NTM, [](int i) { return i; }, E | seq_of(l, PH_MLP), 7);
      mark(l, PH_ROW3, 0);
      if (wave == 0) {
        if (!RPF) params();
        row_resid<D, C::KSM>(xr, p.p1, my_row, bv, lane);
        markv(l, PH_ROW3, 1, xr[0].x);
        row_ln<D>(xr, gv, lv, p.eps, xn_of(2 * l + 2) + (size_t)my_row * D, lane);
      }
      signal(p, E | seq_of(l, PH_ROW3));
      mark(l, PH_ROW3, 3);
    }
  }

  // ---- the LM head for each sequence's last row only (generate_cached reads
  // nothing else of its prefill's logits, gpt2.rs:420-423): a GEMV streaming
  // wte once, workgroup wg taking vocabulary rows [wg VPW, wg VPW + VPW),
  // compute wave w every 4th of them, lane l holding columns 4 (l + 64 u) of
  // a row; batches of 4 rows double-buffered in registers ----
  if (p.lm_last) {
    const int lane = tid0 & 63;
    constexpr int NC = D / 4, RB = 4;
    wait_for(p, M, row_wg, E | seq_of(L - 1, PH_ROW3), 8);
    mark(L, PH_QKV, 0);
    const int VPW = (p.V + G - 1) / G, v0 = wg * VPW, v1 = min(p.V, v0 + VPW);
    const int nr = v1 > v0 + wave ? (v1 - v0 - wave + NCW - 1) / NCW : 0;  // this wave's rows
    u64 bk[LM_LAST_MAX] = {0ull, 0ull, 0ull, 0ull};
    if (cw && nr > 0) {
      float4 xs[LM_LAST_MAX][NU];
#pragma unroll
      for (int sq = 0; sq < LM_LAST_MAX; ++sq)
#pragma unroll
        for (int u = 0; u < NU; ++u)
          xs[sq][u] = sq < S ? ldx4<FRESH>(xn_of(2 * L) + (size_t)(sq * T + T - 1) * D + 4 * min(lane + 64 * u, NC - 1))
                             : make_float4(0.f, 0.f, 0.f, 0.f);
      float4 wa[RB][NU], wb[RB][NU];
      auto load = [&](int b, float4 (&w)[RB][NU]) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          const int v = v0 + wave + NCW * min(RB * b + j, nr - 1);
#pragma unroll
          for (int u = 0; u < NU; ++u) w[j][u] = ldnt4(p.wte + (size_t)v * D + 4 * min(lane + 64 * u, NC - 1));
        }
      };
      auto use = [&](int b, const float4 (&w)[RB][NU]) {
#pragma unroll
        for (int j = 0; j < RB; ++j) {
          const int i = RB * b + j;
          if (i >= nr) break;  // wave-uniform
          const int v = v0 + wave + NCW * i;
#pragma unroll
          for (int sq = 0; sq < LM_LAST_MAX; ++sq) {
            if (sq >= S) break;
            float d = 0.f;
#pragma unroll
            for (int u = 0; u < NU; ++u)
              if (lane + 64 * u < NC)
                d += w[j][u].x * xs[sq][u].x + w[j][u].y * xs[sq][u].y + w[j][u].z * xs[sq][u].z +
                     w[j][u].w * xs[sq][u].w;
            d = wsum(d);  // the whole sum in every lane
            if (lane == sq) *RK_GW(float, p.logits + (size_t)(sq * T + T - 1) * p.V + v) = d;
            const u64 k = argmax_key(d, (uint32_t)v);
            bk[sq] = k > bk[sq] ? k : bk[sq];
          }
        }
      };
      const int nb = (nr + RB - 1) / RB;
      load(0, wa);
      if (nb > 1) load(1, wb);
      for (int b = 0; b < nb; b += 2) {
        use(b, wa);
        if (b + 2 < nb) load(b + 2, wa);
        if (b + 1 < nb) {
          use(b + 1, wb);
          if (b + 3 < nb) load(b + 3, wb);
        }
      }
    }
    // lane s adds sequence s's best key (the same in every lane) to keys[s];
    // the returned value is consumed so that the max has been performed
    // before this workgroup counts itself done
    const u64 b = lane == 0 ? bk[0] : lane == 1 ? bk[1] : lane == 2 ? bk[2] : bk[3];
    if (cw && lane < S && b != 0ull) {
      const u64 prev =
          __hip_atomic_fetch_max(RK_GW(u64, p.keys + lane), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("" : : "v"(prev));
    }
    mark(L, PH_QKV, 3);
  } else
  // ---- tied LM head (gpt2.rs:392-396): logits[r][n] = ln_f(x_r) . wte[n] ----
  // Tiles of 32 vocabulary rows, workgroup wg taking tiles wg, wg + G, ...;
  // each tile in NS = D / 128 k steps, compute wave w taking k [128 s + 32 w,
  // +32) of step s. A wave streams its (tile, step) weight slices (32 rows x
  // 128 bytes) by DMA through a ring of LM_RING LDS slots of its own, so no
  // other wave waits for them; the ln_f rows stay in registers.
  {
    const int lane = tid0 & 63;
    constexpr int NS = D / 128, R = LM_RING;
    const int ntl = (p.V + TN - 1) / TN;
    const int nst = (wg < ntl ? (ntl - 1 - wg) / G + 1 : 0) * NS;  // this workgroup's (tile, step) stream
    float* ring = sm.lmw + wave * R * 1024;
    auto issue = [&](int g) {
      w_dma<16>(ring + 1024 * (g % R), p.wte, D, p.V, (wg + (g / NS) * G) * TN, 128 * (g % NS) + 32 * wave, lane);
    };
    if (cw)
      for (int g = 0; g < R && g < nst; ++g) issue(g);
    wait_for(p, M, row_wg, E | seq_of(L - 1, PH_ROW3), 8);
    mark(L, PH_QKV, 0);
    float4 a[NS][4];
    if (cw) {
#pragma unroll
      for (int st = 0; st < NS; ++st) a_rows<16, FRESH>(a[st], xn_of(2 * L), D, M, 128 * st + 32 * wave + 16 * (lane >> 5), lane);
    }
    u64 best[4] = {0ull, 0ull, 0ull, 0ull};  // argmax keys of this thread's rows (greedy finish)
    for (int g0 = 0; g0 < nst; g0 += NS) {
      floatx16 c0 = {}, c1 = {};
      if (cw) {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
          const int g = g0 + st;
          // slot g has landed once at most the DMAs of the later steps in flight are outstanding
          lm_wait(min(R - 1, nst - 1 - g));
          const float* sl = ring + 1024 * (g % R);
#pragma unroll
          for (int q = 0; q < 4; ++q) mma4(a[st][q], w_chunk<16>(sl, q, lane), c0, c1);
          if (g + R < nst) issue(g + R);
        }
      }
      const int n0 = (wg + (g0 / NS) * G) * TN;
      tile_out(c0 + c1, red, lane, [&](int r, int cc, float v) {
        if (r < M && n0 + cc < p.V) {
          p.logits[(size_t)r * p.V + n0 + cc] = v;
          const u64 k = argmax_key(v, (uint32_t)(n0 + cc));
          best[r & 3] = k > best[r & 3] ? k : best[r & 3];
        }
      });
    }
    if (p.keys != nullptr && cw) {
      // per row: the max over the 32 lanes of its half-wave, one device-scope
      // atomic max per workgroup for each sequence's last row; its returned
      // value is consumed so that the max has been performed before this
      // workgroup counts itself done
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        u64 b = best[u];
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
          const u64 o = __shfl_xor(b, off, 64);
          b = o > b ? o : b;
        }
        const int r = 8 * wave + 4 * (lane >> 5) + u;
        if ((lane & 31) == 0 && r < M && r % T == T - 1 && b != 0ull) {
          const u64 prev = __hip_atomic_fetch_max(RK_GW(u64, p.keys + r / T), b, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
          asm volatile("" : : "v"(prev));
        }
      }
    }
    mark(L, PH_QKV, 3);
  }

  if (tracing && tid0 == 0) {
    const int n = (L + 2) * 32;
    for (int i = 0; i < n; ++i) p.trace[(size_t)wg * TRACE_WORDS + i] = trs[i];
    p.trace[(size_t)wg * TRACE_WORDS + TRACE_WORDS - 1] = t0;
  }
  // the last workgroup to finish advances the epoch for the next launch
  __syncthreads();
  if (tid0 == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(RK_GW(unsigned, p.done), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == G - 1) {
      if (p.keys != nullptr) {
        const int step = *RK_G(int, p.step);
        for (int sq = 0; sq < S; ++sq) {
          const u64 k = __hip_atomic_load(RK_GW(u64, p.keys + sq), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const uint32_t t = argmax_key_index(k);
          p.token[sq] = t;
          if (p.ids_out) p.ids_out[(size_t)sq * p.ld_ids + step] = t;
          p.keys[sq] = 0ull;
        }
        *p.fin_pos = *p.fin_pos + 1;
        *p.step = step + 1;
      }
      __hip_atomic_store(RK_GW(unsigned, p.done), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(RK_GW(u64, p.epoch), (E >> 16) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace rk
}  // namespace rtg
