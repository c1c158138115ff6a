// Device side of the persistent decode step (batch 1), templated on the model
// width D, vocabulary V and weight storage WT so that every segment count and
// row split is a compile-time constant. Included by the per-size
// instantiation files; see decode_persistent.hip for the host side.
//
// One cooperative launch runs a whole forward_cached(&[token]) + argmax
// (rusttorch-core/src/nn/gpt2.rs:358-399, 858-868) on all 256 CUs:
//  * Every weight matrix is streamed once per step. Workgroup w owns the
//    output rows [w*RPW, (w+1)*RPW) of every phase; its GEMV waves hold their
//    share of a phase's weights in registers, loaded one phase ahead into two
//    alternating buffers, so HBM keeps streaming while workgroups exchange
//    activations.
//  * Workgroups exchange activations without grid barriers or agent-scope
//    fences (~1-2 us each on this part): each published value is a 64-bit
//    word {tag, f32} written with one relaxed agent-scope atomic store, and
//    readers poll until every tag equals the step's epoch. Each (layer, phase)
//    has its own buffer, so a word is written once per step and never
//    overwritten while someone may still read it.
//  * Waves are specialised so that no wave holding in-flight weight loads
//    ever has to drain them for a publication:
//      wave 0         leader: LayerNorm statistics, epilogues, stores;
//                     polls the attention's q/k/v; attention rows
//      waves 1..NA    helpers: poll inputs with the leader; attention rows
//      waves NA+1..   GEMV waves: weights in registers, dot products
//    Leader/helpers and GEMV waves meet only through LDS counters, and all
//    pointers are address-space qualified so no flat access ties the LDS
//    counter (lgkmcnt) to global loads.
//  * Every wait is bounded; a timeout sets *err and lets the step finish with
//    wrong numbers instead of hanging; the host turns *err into an error.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "argmax_key.h"
#include "kernels.h"

namespace rtg {
namespace pk {

#ifndef PK_PACE
#define PK_PACE 12
#endif

constexpr int G = 256;              // workgroups = CUs of an MI355X
// 8 waves per workgroup = 2 per SIMD, which leaves 256 VGPRs per wave for the
// two register-resident weight buffers.
constexpr int NA = 2;               // helper waves
constexpr int NC = 5;               // GEMV waves
constexpr int NGLUE = 1 + NA;       // leader + helpers
constexpr int NATT = NGLUE;         // attention waves: the leader and the helpers
constexpr int NTHREADS = (1 + NA + NC) * 64;
constexpr int HD = 64;              // head_dim of every GPT-2 size
constexpr int CMAX = 16;            // attention chunks per head
constexpr int ITEM_WORDS = HD + 2;  // o[64], m, l
constexpr int MAX_ITEMS = G;        // heads * chunks: at most one attention item per workgroup
constexpr int PART_MAX = 1536;      // segment partials per workgroup
// GEMV phase types, each with its own input-ready counter. A glue wave counts
// itself once per layer in each; every workgroup owns rows of the FC phase in
// every supported shape, so no wave can run a whole layer ahead of another and
// a count of NGLUE * (l + 1) means that every glue wave delivered layer l.
enum { PH_QKV = 0, PH_PROJ = 1, PH_FC = 2, PH_MLP = 3, PH_LM = 4 };
constexpr int KVS = 120;            // cached positions of one item staged in LDS (NATT windows)
// Exchange layout: each producer owns a slot of whole 128-byte lines, so no
// two producers ever write the same line and readers of one producer's words
// touch only that producer's lines (lines written by many producers and read
// by all 256 workgroups were measured to double the exchange latency).
constexpr int LINE_WORDS = 16;  // u64 words per 128-byte line
__host__ __device__ constexpr int slot_words(int rows) { return (rows + LINE_WORDS - 1) / LINE_WORDS * LINE_WORDS; }
constexpr int ITEM_SLOT = slot_words(ITEM_WORDS);  // words of one attention item's slot
constexpr unsigned SPIN_CAP = 1u << 21;

typedef unsigned long long u64;

#define PK_G(T, p) ((const __attribute__((address_space(1))) T*)(p))
#define PK_GW(T, p) ((__attribute__((address_space(1))) T*)(p))
#define PK_C(T, p) ((const __attribute__((address_space(4))) T*)(p))

struct LayerPtrs {
  const void *wqkv, *waproj, *wfc, *wmproj;
  const float *bqkv, *baproj, *bfc, *bmproj, *ln1w, *ln1b, *ln2w, *ln2b;
  // LayerNorm folded into the following GEMV (computed once at load time):
  // for output row r, s[r] = sum_k W[r][k] g[k] and c[r] = bias[r] +
  // sum_k W[r][k] b[k], so with the GEMV input centred on a value c0 known
  // ahead (the mean of the previous LayerNorm's input),
  // LN(x) @ W + bias = inv_std * (W.((x - c0) g) - (mean - c0) s) + c:
  // only the drift of the mean between two LayerNorms is subtracted.
  const float *sq, *cq, *sf, *cf;
};

struct Params {
  const LayerPtrs* layers;
  const void* wte;
  const float *wpe, *lnfw, *lnfb;
  const float *sl, *cl;  // ln_f folded into the tied LM head, as for the layers
  int L, P;
  int V;  // vocabulary rows of the LM head (at most the instance's compiled V; the rows go to the first
          // ceil(V / RPW) workgroups)
  float eps;
  float* kc;  // [L][H][P][HD]
  float* vc;
  long kv_layer;  // floats per layer
  uint32_t* token;  // current token in; the argmax token out (written by the last workgroup)
  int* pos;         // position of the current token; advanced by the last workgroup
  uint32_t* ids_out;  // generated ids (ids_out[*step] = argmax token)
  int* step;
  unsigned* done;     // arrivals of workgroups at the end of the step (reset by the last)
  unsigned* epoch;  // tag of this step; advanced by the last workgroup
  u64* tag;  // tagged words, lw per layer
  long lw;
  int o_qkv, o_att, o_head, o_x2, o_h, o_x3;  // exchange regions of a layer (words)
  float* logits;
  u64* keys;
  unsigned* err;
  u64* trace;         // optional: per-workgroup timestamps (TRACE_STRIDE entries each)
  const void* dummy;  // >= 1 KiB of zeros: target of the loads of segments a wave does not own
  // Test hook (test_spins > 0): layer 1's x3 fetch waits for a tag no
  // producer writes and gives up after test_spins polling rounds, so the
  // step takes its timeout path (error word) without a fault or hang.
  unsigned test_spins;
};

// Optional phase trace (p.trace != null): timestamps of the 100 MHz constant
// clock relative to the workgroup's start, kept in LDS so that tracing adds
// no global stores (and no memory-counter waits) to the traced paths, and
// written to p.trace[wg * TRACE_STRIDE + idx] (absolute, u64) at the end.
// Index spaces: [0, 16L+4) layer/LM-head points of the leader, 800 + 4l + k
// helper/LayerNorm points, 1024 + 2*seq (+1) GEMV start/end of phase seq.
constexpr int TRACE_STRIDE = 2048;
constexpr int TRACE_N = 1536;
#define PK_TRACE(p, idx, lane)                                               \
  do {                                                                       \
    if ((p).trace && (lane) == 0 && (idx) >= 0 && (idx) < TRACE_N)           \
      sm.trace_rel[(idx)] = (unsigned)(wall_clock64() - sm.trace_t0) | 1u;   \
  } while (0)

// Row split of one GEMV phase: N outputs, each a dot product over K inputs
// stored as VR 16-byte vectors; a segment = 64 vectors of one row. The rows
// go to the first GW_ workgroups (RPW each); the others own none.
template <int N_, int K_, int E_, int SPW_ = 0, int GW_ = G>
struct Geom {
  static constexpr int N = N_, K = K_, VR = K_ / E_, SPR = (VR + 63) / 64;
  static constexpr int RPW = (N_ + GW_ - 1) / GW_;  // rows of each of the first GW_ workgroups
  static constexpr int SW = slot_words(RPW);  // exchange slot of one workgroup's rows
  static constexpr int SEGS = RPW * SPR;
  // Segments per GEMV wave: an even split, rounded up to whole rows unless
  // that would exceed max(12, even split) registers-worth of segments, so
  // that each wave reduces whole rows with a compile-time structure.
  static constexpr int SPW0 = (SEGS + NC - 1) / NC;
  static constexpr int SPW_ROWS = (SPW0 + SPR - 1) / SPR * SPR;
  static constexpr int SPW = SPW_ ? SPW_ : SPW_ROWS <= (SPW0 > 12 ? SPW0 : 12) ? SPW_ROWS : SPW0;
  static constexpr bool ALIGNED = SPW % SPR == 0;  // every wave starts on a row
};

constexpr int cmax(int a, int b) { return a > b ? a : b; }

template <int D_, int V_, int WT_>
struct Cfg {
  static constexpr int D = D_, V = V_, WT = WT_, H = D_ / HD, E = WT_ == W_BF16 ? 8 : 4;
  // refill pacing (seg_issue): measured best at 4 for d = 768 with the
  // cache policy below (c1: 203.2-203.8 µs per token against 203.6-203.9 at
  // 2, 204.1-204.7 at 8, 209.9 at 12, 211.3 without pacing) and at 6 for
  // d = 1024 (c3: 582.5 µs against 582.8 at 4, 593 at 8, 590.5 at 12, 594
  // at 2); 12 elsewhere
  static constexpr int PACE = D_ == 768 ? 4 : D_ == 1024 ? 6 : PK_PACE;
  // Cache policy of the weight loads. Matrices loaded with normal loads stay
  // in the 256 MB last-level cache from one step to the next; the others
  // are loaded non-temporally (~15% faster streaming, not kept). Their
  // refills run during the exchanges (c_attn's during the h exchange, the
  // projections' during x3 and x2), which then compete with less HBM
  // traffic. d = 768: c_attn, attention projection and MLP projection
  // (226 MB; wte and c_fc non-temporal): c1 202.5-202.8 µs per token; with
  // c_fc instead of the MLP projection 202.5-202.7; c_attn alone beside a
  // cached wte 205.6-206.5; wte alone 210.6; all four matrices (340 MB)
  // 212.6. The multi-row forward reads the same matrices and gains too
  // (c1 prefill 0.413-0.420 against 0.418-0.423 ms). d = 1024: the
  // attention projections (100 MB): c3 574.6 against 578.5 µs (c_attn,
  // 302 MB: 588.4).
  static constexpr bool Q_NT = D_ != 768, P_NT = D_ != 768 && D_ != 1024, M_NT = D_ != 768;
  typedef Geom<3 * D, D, E> GQ;
  // the attention projection on the first D / 8 workgroups, 8 rows each: its
  // input then goes to (and x2 comes from) 96 workgroups at d = 768 instead
  // of 256 (c1: 209.5 against 215.5 µs per token; 4 rows: 215.5, 6: 211.6,
  // 12: 210.0, 16: 212.1; c3: 591 against 596.5)
  typedef Geom<D, D, E, 0, (D + 7) / 8> GP;
  typedef Geom<4 * D, D, E> GF;
  typedef Geom<D, 4 * D, E> GM;
  static constexpr int MAXSEG = cmax(cmax(GQ::SPW, GP::SPW), cmax(GF::SPW, GM::SPW));
  typedef Geom<V, D, E, MAXSEG> GL;  // LM head, streamed in chunks of MAXSEG per wave
  static_assert(D % HD == 0 && D <= 1600, "model width");
  static_assert(GQ::RPW <= 64 && GP::RPW <= 64 && GF::RPW <= 64 && GM::RPW <= 64, "one bias per leader lane");
  static_assert(GQ::SEGS <= PART_MAX && GF::SEGS <= PART_MAX && GM::SEGS <= PART_MAX && GL::SEGS <= PART_MAX,
                "segment partials exceed LDS");
  static_assert(H <= MAX_ITEMS, "heads");
};

template <int D>
struct Smem {
  float in_vec[2][4 * D];  // GEMV input, double-buffered by phase parity
  float xraw[D];           // residual input of the current layer
  float x2raw[2][D];       // residual after attention, by layer parity (read one layer later as a centre)
  float part[PART_MAX];
  float stage[CMAX * ITEM_WORDS];  // a chunked head's items, on the workgroup that merges them
  float kv_k[KVS * HD], kv_v[KVS * HD];  // K/V rows [j0, j0 + KVS) of this workgroup's item
  float att_part[NATT][ITEM_WORDS];
  float att_q[HD], att_k[HD], att_v[HD];
  // in_ready[phase]: +1 per glue wave once its share of that phase's GEMV
  // input is in LDS (one counter per phase type, see PH_QKV..PH_LM);
  // gemv_done: +1 per GEMV wave per phase; glue_cnt: glue-wave barrier;
  // att_go: layers whose q/k/v the leader has put in LDS; att_cnt: attention
  // waves that finished the layer's attention.
  unsigned in_ready[5], gemv_done, glue_cnt, att_go, att_cnt;
  u64 trace_t0;
  unsigned trace_rel[TRACE_N];
};

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ u64 tload(const u64* p) {
  return __hip_atomic_load(PK_GW(u64, p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(u64* p, float v, unsigned tag) {
  __hip_atomic_store(PK_GW(u64, p), ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// Native vector types for address-space qualified loads (HIP's float4 class
// does not copy from an address-space qualified object).
typedef float f4v __attribute__((ext_vector_type(4)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4g(const float* p) {
  const f4v v = PK_G(f4v, p)[0];
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ unsigned lds_load(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(unsigned* p, unsigned v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Order this wave's LDS accesses (lgkmcnt only).
__device__ __forceinline__ void lds_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local"); }
__device__ __forceinline__ void lds_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local"); }

__device__ __forceinline__ bool err_set(const unsigned* err) {
  return __hip_atomic_load(PK_GW(unsigned, err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void raise_err(unsigned* err, unsigned code) {
  __hip_atomic_fetch_or(PK_GW(unsigned, err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin (whole wave) until *p >= target (LDS counter). Bounded.
__device__ __forceinline__ void lds_wait_ge(unsigned* p, unsigned target, unsigned* err) {
  unsigned spins = 0;
  while (lds_load(p) < target) {
    __builtin_amdgcn_s_sleep(1);
    if (++spins > (SPIN_CAP << 3)) {
      raise_err(err, 2u);
      break;
    }
  }
  lds_acquire();
}

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// DPP lane move within 16-lane rows (quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] =
// 0x4E, row_ror:4 = 0x124, row_ror:8 = 0x128): four of them sum a row.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Combine each lane's value with the lane 16 (or 32) apart through gfx950's
// v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip): the two
// swapped registers hold the lane's own value and its partner's, so their sum
// (max) is the pairwise sum (max), identical in both lanes.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// exp(x) for the softmax, x <= 0: 2^(x log2 e) on the hardware exponent
// (v_exp_f32, about 1 ulp; exp(-inf) = 0) instead of the libm-accurate
// sequence, which costs ~15 instructions per call on the attention's critical
// path; the difference to the reference's f32 exp is far inside the logits
// tolerance.
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// gelu_new, gpt2.rs:837-847 (the reference's association).
__device__ __forceinline__ float gelu_new(float x) {
  const float sqrt_2_pi = 0.7978845608028654f;
  float inner = sqrt_2_pi * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <int WT>
struct V16;
template <>
struct V16<W_F32> {
  typedef f4v T;
  static constexpr int E = 4;
  // the 16-byte quads of x one weight vector pairs with, and their dot product
  static constexpr int XQ = 1;
  __device__ __forceinline__ static void load_x(float4 (&xq)[XQ], const float* x) {
    xq[0] = *reinterpret_cast<const float4*>(x);
  }
  __device__ __forceinline__ static float dot(const T& w, const float4 (&xq)[XQ]) {
    return w.x * xq[0].x + w.y * xq[0].y + w.z * xq[0].z + w.w * xq[0].w;
  }
};
template <>
struct V16<W_BF16> {
  typedef u4v T;
  static constexpr int E = 8;
  // bf16_to_f32 = bits << 16 (nn/safetensors.rs:389-391)
  // the 16-byte quads of x one weight vector pairs with, and their dot product
  static constexpr int XQ = 2;
  __device__ __forceinline__ static void load_x(float4 (&xq)[XQ], const float* x) {
    xq[0] = *reinterpret_cast<const float4*>(x);
    xq[1] = *reinterpret_cast<const float4*>(x + 4);
  }
  __device__ __forceinline__ static float dot(const T& w, const float4 (&xq)[XQ]) {
    const float4 a = xq[0], c = xq[1];
    float s = __uint_as_float(w.x << 16) * a.x + __uint_as_float(w.x & 0xffff0000u) * a.y;
    s += __uint_as_float(w.y << 16) * a.z + __uint_as_float(w.y & 0xffff0000u) * a.w;
    s += __uint_as_float(w.z << 16) * c.x + __uint_as_float(w.z & 0xffff0000u) * c.y;
    s += __uint_as_float(w.w << 16) * c.z + __uint_as_float(w.w & 0xffff0000u) * c.w;
    return s;
  }
};

// ---------------------------------------------------------------------------
// GEMV waves. Wave cw of workgroup wg handles workgroup segments
// [seg_base + cw*SPW, seg_base + (cw+1)*SPW). All bookkeeping is scalar.
// ---------------------------------------------------------------------------

// PACE > 0: sleep up to PACE*64 clocks between loads while the wave's next
// input is not ready yet (*ready < next), so a refill does not flood this
// CU's memory queue ahead of the exchanges; the sleep is cut short (to 128
// clocks) once the input is ready, after which the remaining loads go out
// back to back. The pacing is the only conditional part: the loads stay in
// fixed order.
#ifndef PK_W_NT
#define PK_W_NT 1
#endif
template <int WT, int MAXSEG, class GEO, int PACE = PK_PACE, bool NT = PK_W_NT>
__device__ __forceinline__ void seg_issue(typename V16<WT>::T (&buf)[MAXSEG], const void* W, const void* dummy, int wg,
                                          int cw, int lane, int seg_base, unsigned* ready = nullptr,
                                          unsigned next = 0, int n_rows = GEO::N) {
  typedef typename V16<WT>::T Vec;
  const int row0 = wg * GEO::RPW;
  const int rows_here = min(GEO::RPW, n_rows - row0);
  const int segs_here = rows_here > 0 ? rows_here * GEO::SPR : 0;
  const int s0 = seg_base + cw * GEO::SPW;
  const int nseg = min(GEO::SPW, segs_here - s0);
  int lr = s0 / GEO::SPR, j = s0 - lr * GEO::SPR;
  const Vec* base = reinterpret_cast<const Vec*>(W) + (long)row0 * GEO::VR;
  bool go = false;  // the input was seen ready: no more pacing (nor LDS reads)
  // Branch-free: the compiler's wait-count analysis then sees a fixed load
  // order and waits only for the buffer being consumed. Segments this wave
  // does not own read a small zero page instead (L2-resident).
#pragma unroll
  for (int i = 0; i < MAXSEG; ++i) {
    if (i < GEO::SPW) {
      const Vec* rowp = i < nseg ? base + (long)lr * GEO::VR + j * 64 : reinterpret_cast<const Vec*>(dummy);
      const int li = (GEO::VR % 64 == 0) ? lane : min(lane, max(0, min(GEO::VR - j * 64, 64) - 1));
      // non-temporal: weights are streamed once per step (measured ~15% more
      // streaming bandwidth than plain loads on this part)
      if constexpr (NT) buf[i] = __builtin_nontemporal_load(PK_G(Vec, rowp) + li);
      else buf[i] = PK_G(Vec, rowp)[li];
      if (PACE > 0 && i + 1 < GEO::SPW && !go)
        for (int t = 0; t < PACE / 2; ++t) {
          if (lds_load(ready) >= next) {
            go = true;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
        }
    }
    if (++j == GEO::SPR) {
      j = 0;
      ++lr;
    }
  }
}

// Sum over the wave, in every lane: DPP within each 16-lane row, then the
// permlane swaps across rows (VALU only, no readlane or LDS, so independent
// sums interleave).
__device__ __forceinline__ float wave_sum_all(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  return xor32_sum(xor16_sum(v));
}

// The wave's segments [s0, s0 + SPW) cover pieces of at most NPC rows (whole
// rows when the geometry is aligned). Every segment's products are summed
// lane-wise per piece, each piece's lane sums reduced over the wave (the
// NPC reductions independent of each other), and lane k < SPW then writes
// slot s0 + k: its piece's sum if segment k ends the piece, else 0, so that a
// row's slots add up to its dot product.
template <int WT, int MAXSEG, class GEO>
__device__ __forceinline__ void seg_compute(const typename V16<WT>::T (&buf)[MAXSEG], const float* x, float* part,
                                            int wg, int cw, int lane, int seg_base, int n_rows = GEO::N) {
  constexpr int E = V16<WT>::E, SPR = GEO::SPR, SPW = GEO::SPW;
  constexpr int NPC = GEO::ALIGNED ? SPW / SPR : (SPW + SPR - 2) / SPR + 1;
  const int row0 = wg * GEO::RPW;
  const int rows_here = min(GEO::RPW, n_rows - row0);
  const int segs_here = rows_here > 0 ? rows_here * SPR : 0;
  const int s0 = seg_base + cw * SPW;
  const int nseg = min(SPW, segs_here - s0);
  const int j0 = GEO::ALIGNED ? 0 : s0 % SPR;  // aligned: every wave range starts a row
  // x of every segment first (the LDS reads in flight together) where that
  // takes at most 64 registers, else segment by segment (wider bf16 shapes
  // would spill)
  constexpr int XQ = V16<WT>::XQ;
  constexpr bool PRE = MAXSEG * XQ * 4 <= 64;
  float4 xq[PRE ? MAXSEG : 1][XQ];
  if constexpr (PRE) {
#pragma unroll
    for (int i = 0; i < MAXSEG; ++i)
      if (i < SPW) V16<WT>::load_x(xq[i], x + min(((j0 + i) % SPR) * 64 + lane, GEO::VR - 1) * E);
  }
  float r[NPC];
#pragma unroll
  for (int q = 0; q < NPC; ++q) r[q] = 0.f;
#pragma unroll
  for (int i = 0; i < MAXSEG; ++i) {
    if (i < SPW) {
      const int v = ((j0 + i) % SPR) * 64 + lane;
      if constexpr (!PRE) V16<WT>::load_x(xq[0], x + min(v, GEO::VR - 1) * E);
      const float d = v < GEO::VR ? V16<WT>::dot(buf[i], xq[PRE ? i : 0]) : 0.f;
      if constexpr (GEO::ALIGNED) {
        r[i / SPR] += d;
      } else {
        const int pc = (j0 + i) / SPR;
#pragma unroll
        for (int q = 0; q < NPC; ++q) r[q] += pc == q ? d : 0.f;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NPC; ++q) r[q] = wave_sum_all(r[q]);
  if (lane < SPW && lane < nseg) {
    const int pc = (j0 + lane) / SPR;
    const bool ends = (j0 + lane) % SPR == SPR - 1 || lane == SPW - 1;
    float val = 0.f;
#pragma unroll
    for (int q = 0; q < NPC; ++q) val = pc == q ? r[q] : val;
    part[s0 + lane] = ends ? val : 0.f;
  }
}

template <class C>
__device__ __forceinline__ void gemv_role(const Params& p, Smem<C::D>& sm, int cw, int lane) {
  constexpr int WT = C::WT, MS = C::MAXSEG;
  typedef typename V16<WT>::T Vec;
  typedef typename C::GQ GQ;
  typedef typename C::GP GP;
  typedef typename C::GF GF;
  typedef typename C::GM GM;
  typedef typename C::GL GL;
  const int wg = blockIdx.x;
  Vec A[MS], B[MS];
  unsigned seq = 0;
  const void* dz = p.dummy;
  // Layer pointers come through scalar loads (constant address space): a
  // vector load would need a vmcnt wait that also drains the prefetch.
  const __attribute__((address_space(4))) LayerPtrs* LP = PK_C(LayerPtrs, p.layers);
  // The code below issues every buffer refill unconditionally (the last
  // layer is peeled) so each consume waits only for its own buffer.
  auto compute_and_signal = [&](auto& buf, const float* x, auto geo_tag, int ph, int l) {
    typedef decltype(geo_tag) GEO;
    lds_wait_ge(&sm.in_ready[ph], (unsigned)(l + 1) * NGLUE, p.err);
    ++seq;
    if (cw == 0) PK_TRACE(p, 1024 + 2 * (int)seq, lane);
    // raised issue priority over the glue waves sharing the SIMD, which poll
    // the next exchange meanwhile (c1: 215.1 against 217.2 µs per token)
    __builtin_amdgcn_s_setprio(2);
    seg_compute<WT, MS, GEO>(buf, x, sm.part, wg, cw, lane, 0);
    __builtin_amdgcn_s_setprio(0);
    if (cw == 0) PK_TRACE(p, 1025 + 2 * (int)seq, lane);
    lds_release();
    if (lane == 0) lds_add(&sm.gemv_done, 1);
  };
  seg_issue<WT, MS, GQ, 0, C::Q_NT>(A, LP[0].wqkv, dz, wg, cw, lane, 0);  // needed first: no pacing
  // each refill is paced until the input of this wave's next compute is ready
  auto rdy = [&](int ph) { return &sm.in_ready[ph]; };
  seg_issue<WT, MS, GP, C::PACE, C::P_NT>(B, LP[0].waproj, dz, wg, cw, lane, 0, rdy(PH_QKV), NGLUE);
  for (int l = 0; l + 1 < p.L; ++l) {
    const unsigned n1 = (unsigned)(l + 1) * NGLUE;
    compute_and_signal(A, sm.in_vec[1], GQ(), PH_QKV, l);   // QKV; refill A with FC
    seg_issue<WT, MS, GF, C::PACE>(A, LP[l].wfc, dz, wg, cw, lane, 0, rdy(PH_PROJ), n1);
    compute_and_signal(B, sm.in_vec[0], GP(), PH_PROJ, l);  // attention projection; refill B with MLP projection
    seg_issue<WT, MS, GM, C::PACE, C::M_NT>(B, LP[l].wmproj, dz, wg, cw, lane, 0, rdy(PH_FC), n1);
    compute_and_signal(A, sm.in_vec[1], GF(), PH_FC, l);    // FC; refill A with next QKV
    seg_issue<WT, MS, GQ, C::PACE, C::Q_NT>(A, LP[l + 1].wqkv, dz, wg, cw, lane, 0, rdy(PH_MLP), n1);
    compute_and_signal(B, sm.in_vec[0], GM(), PH_MLP, l);   // MLP projection; refill B with next attention projection
    seg_issue<WT, MS, GP, C::PACE, C::P_NT>(B, LP[l + 1].waproj, dz, wg, cw, lane, 0, rdy(PH_QKV), n1 + NGLUE);
  }
  {  // last layer: the refills after FC / MLP projection are the LM head's chunks 0 and 1
    const int l = p.L - 1;
    const unsigned n1 = (unsigned)(l + 1) * NGLUE;
    compute_and_signal(A, sm.in_vec[1], GQ(), PH_QKV, l);
    seg_issue<WT, MS, GF, C::PACE>(A, LP[l].wfc, dz, wg, cw, lane, 0, rdy(PH_PROJ), n1);
    compute_and_signal(B, sm.in_vec[0], GP(), PH_PROJ, l);
    seg_issue<WT, MS, GM, C::PACE, C::M_NT>(B, LP[l].wmproj, dz, wg, cw, lane, 0, rdy(PH_FC), n1);
    compute_and_signal(A, sm.in_vec[1], GF(), PH_FC, l);
    seg_issue<WT, MS, GL, C::PACE>(A, p.wte, dz, wg, cw, lane, 0, rdy(PH_MLP), n1, p.V);
    compute_and_signal(B, sm.in_vec[0], GM(), PH_MLP, l);
    seg_issue<WT, MS, GL, C::PACE>(B, p.wte, dz, wg, cw, lane, NC * GL::SPW, rdy(PH_LM), NGLUE, p.V);
  }
  // LM head (tied wte, gpt2.rs:392-396): chunk c = workgroup segments
  // [c*NC*SPW, (c+1)*NC*SPW), alternating between A and B.
  lds_wait_ge(&sm.in_ready[PH_LM], NGLUE, p.err);
  ++seq;
  constexpr int PER_CHUNK = NC * GL::SPW;
  const int rows_here = min(GL::RPW, p.V - wg * GL::RPW);
  const int segs_here = rows_here > 0 ? rows_here * GL::SPR : 0;
  for (int base = 0; base < segs_here; base += 2 * PER_CHUNK) {
    // nothing else is in flight now: stream at full rate
    seg_compute<WT, MS, GL>(A, sm.in_vec[1], sm.part, wg, cw, lane, base, p.V);
    seg_issue<WT, MS, GL, 0>(A, p.wte, dz, wg, cw, lane, base + 2 * PER_CHUNK, nullptr, 0, p.V);
    seg_compute<WT, MS, GL>(B, sm.in_vec[1], sm.part, wg, cw, lane, base + PER_CHUNK, p.V);
    seg_issue<WT, MS, GL, 0>(B, p.wte, dz, wg, cw, lane, base + 3 * PER_CHUNK, nullptr, 0, p.V);
  }
  lds_release();
  if (lane == 0) lds_add(&sm.gemv_done, 1);
}

// ---------------------------------------------------------------------------
// Leader + helper waves ("glue").
// ---------------------------------------------------------------------------

template <int D>
__device__ __forceinline__ void glue_barrier(Smem<D>& sm, unsigned& gen, int lane, unsigned* err) {
  ++gen;
  lds_release();
  if (lane == 0) lds_add(&sm.glue_cnt, 1);
  lds_wait_ge(&sm.glue_cnt, gen * NGLUE, err);
}

// Address of word i of an exchange whose producers each publish RPW words
// into slots of SW words.
template <int RPW, int SW>
__device__ __forceinline__ int slot_of(int i) {
  return (i / RPW) * SW + i % RPW;
}

// Mean of the D floats x (LDS) on one wave: a lane's D / 64 values summed in
// order, then the fixed wave reduction; every wave gets the same value.
template <int D>
__device__ __forceinline__ float lds_mean(const float* x, int lane) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < D / 64; ++k) s += x[lane + 64 * k];
  return wave_sum_all(s) / (float)D;
}

// All glue lanes fetch the n tagged words of an exchange into dst: every
// word is read with a coherent load (never a stale line of this XCD's L2)
// and stale words are re-read until their tags equal the step's epoch. The
// data is polled directly: with one line per producer slot, a poll costs
// the same line requests as polling a per-producer flag would, and saves
// the flag's extra round trip. The NW = ceil(NMAX / 192) words of a lane in
// a chunk of NMAX words are in flight together, so an exchange of n <= NMAX
// words costs one polling round trip; longer ones take n / NMAX. A stale
// word is re-read as soon as its round returns (c1: 227.3 µs per token
// against 228.2 with a 64-clock sleep between rounds, 232.7 with 512; two
// staggered rounds in flight per word: 252 µs). With SCALE,
// dst2[i] = word * g[i] as well (the LayerNorm gain applied to a GEMV input
// whose LayerNorm is folded).
// With SCALE the GEMV input is also centred: dst2[i] = (word - c0) * g[i],
// c0 = the mean of the D floats at cen_src (the previous LayerNorm's input,
// in LDS once *rdy >= rdy_n), computed by every glue wave alike while its
// first polling round is in flight, and returned in *c0.
template <int RPW, int SW, int NMAX, bool SCALE = false, int D = 0>
__device__ __forceinline__ void glue_fetch(const u64* src, int n, unsigned tag, float* dst, int gl, unsigned* err,
                                           float* dst2 = nullptr, const float* g = nullptr,
                                           const float* cen_src = nullptr, unsigned* rdy = nullptr,
                                           unsigned rdy_n = 0, float* c0 = nullptr, unsigned cap = SPIN_CAP) {
  constexpr int NG = NGLUE * 64;
  constexpr int NW = (NMAX + NG - 1) / NG;
  static_assert(!SCALE || (NMAX >= D && D % 64 == 0), "a centred fetch is one polling round over D words");
  float cen = 0.f;
  for (int base = 0; base < n; base += NW * NG) {
    float gv[NW];
    if constexpr (SCALE) {
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int i = base + gl + k * NG;
        gv[k] = i < n ? PK_G(float, g)[i] : 0.f;
      }
    }
    u64 w[NW];
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const int i = base + gl + k * NG;
      w[k] = i < n ? tload(src + slot_of<RPW, SW>(i)) : ((u64)tag << 32);
    }
    if constexpr (SCALE) {
      lds_wait_ge(rdy, rdy_n, err);
      cen = lds_mean<D>(cen_src, gl & 63);
      *c0 = cen;
    }
    unsigned spins = 0;
    for (;;) {
      bool all = true;
#pragma unroll
      for (int k = 0; k < NW; ++k)
        if ((unsigned)(w[k] >> 32) != tag) all = false;
      if (all) break;
      if (++spins > cap || ((spins & 255u) == 0u && err_set(err))) {
        raise_err(err, 1u);
        break;
      }
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int i = base + gl + k * NG;
        if (i < n && (unsigned)(w[k] >> 32) != tag) w[k] = tload(src + slot_of<RPW, SW>(i));
      }
    }
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const int i = base + gl + k * NG;
      if (i < n) {
        const float v = __uint_as_float((unsigned)w[k]);
        dst[i] = v;
        if constexpr (SCALE) dst2[i] = (v - cen) * gv[k];
      }
    }
  }
}

// A glue wave's share of the input of a GEMV phase of type ph is in LDS.
template <int D>
__device__ __forceinline__ void glue_input_done(Smem<D>& sm, int ph, int lane) {
  lds_release();
  if (lane == 0) lds_add(&sm.in_ready[ph], 1);
}

// Leader only: LayerNorm statistics of src[D] (gpt2.rs:636-666, two-pass:
// mean = sum/n, var = sum((x - mean)^2)/n, inv_std = 1/sqrt(var + eps)). The
// normalisation itself is folded into the following GEMV.
template <int D>
__device__ __forceinline__ void leader_ln_stats(const float* src, float eps, float& mean, float& inv_std, int lane) {
  constexpr int NK = D / 64;
  float x[NK];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    x[k] = src[lane + 64 * k];
    s += x[k];
  }
  mean = wave_sum_all(s) / (float)D;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const float t = x[k] - mean;
    v += t * t;
  }
  const float var = wave_sum_all(v) / (float)D;
  inv_std = 1.0f / sqrtf(var + eps);
}

// ---------------------------------------------------------------------------
// Attention of one item on the NATT glue waves. Wave hw owns cached rows
// [h0, h1) of the item's head and processes them in windows of KVW rows held
// in its own part of the LDS stage.
// ---------------------------------------------------------------------------
constexpr int KVW = KVS / NATT;  // rows of one attention wave's LDS window
// stage_rows fills a window in groups of 4 rows (one 1-KiB LDS-DMA
// instruction each), so a window must hold a whole number of groups
static_assert(KVW % 4 == 0 && KVW * NATT == KVS, "attention window");

// Copy K/V rows [r0, r0 + n), n <= KVW, into a wave's LDS window with
// LDS-direct loads (global_load_lds_dwordx4: lane i of an instruction fills
// bytes [16i, 16i + 16) after the wave-uniform LDS address), so no registers
// are held while the rows are in flight; the wave's own s_waitcnt vmcnt(0)
// makes them readable by that wave. The last instruction repeats row
// r0 + n - 1 into the unused rows of the window.
__device__ __forceinline__ void stage_rows(const float* Kh, const float* Vh, int r0, int n, float* ldsK, float* ldsV,
                                           int lane) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  const int off = (lane & 15) * 4;
  for (int i = 0; 4 * i < n; ++i) {
    const long row = min(r0 + 4 * i + (lane >> 4), r0 + n - 1);
    __builtin_amdgcn_global_load_lds(PK_G(void, Kh + row * HD + off), (lds_ptr)(ldsK + 4 * i * HD), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(PK_G(void, Vh + row * HD + off), (lds_ptr)(ldsV + 4 * i * HD), 16, 0, 0);
  }
}

__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0f70); }  // vmcnt(0) only

// Sum over the 16 lanes of one DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);
  v += dpp_mov<0x128>(v);
  return v;
}

// Online-softmax update of (m, lsum, o4) with the n rows (1 <= n <= KVW) of a
// wave's LDS window (gpt2.rs:796-830: scores q.k / sqrt(64), softmax, p.V).
// 16 lanes per row (4 dims each), 4 rows per wave instruction; lane (grp, dq)
// accumulates lsum and o4 over rows 4t + grp, summed over grp by the caller.
// AT row groups of 4 (n <= 4 * AT); straight-line code so that all LDS reads
// of a loop are in flight together.
template <int AT>
__device__ __forceinline__ void att_window_t(const float* ldsK, const float* ldsV, int n, const float4& q4, int grp,
                                             int dq, float& m, float& lsum, float4& o4) {
  const float scale = 0.125f;  // 1 / sqrt(64)
  float4 k[AT];
#pragma unroll
  for (int t = 0; t < AT; ++t) k[t] = *reinterpret_cast<const float4*>(ldsK + min(4 * t + grp, n - 1) * HD + dq);
  float s[AT];
  float mb = -INFINITY;
#pragma unroll
  for (int t = 0; t < AT; ++t) {
    const float dot = row16_sum(q4.x * k[t].x + q4.y * k[t].y + q4.z * k[t].z + q4.w * k[t].w);
    s[t] = 4 * t + grp < n ? dot * scale : -INFINITY;
    mb = fmaxf(mb, s[t]);
  }
  mb = xor32_max(xor16_max(mb));
  const float mn = fmaxf(m, mb);
  const float corr = m == -INFINITY ? 0.f : fexp(m - mn);
  lsum *= corr;
  o4.x *= corr;
  o4.y *= corr;
  o4.z *= corr;
  o4.w *= corr;
#pragma unroll
  for (int t = 0; t < AT; ++t) {
    const float pj = s[t] == -INFINITY ? 0.f : fexp(s[t] - mn);
    const float4 v = *reinterpret_cast<const float4*>(ldsV + min(4 * t + grp, n - 1) * HD + dq);
    lsum += pj;
    o4.x += pj * v.x;
    o4.y += pj * v.y;
    o4.z += pj * v.z;
    o4.w += pj * v.w;
  }
  m = mn;
}
__device__ __forceinline__ void att_window(const float* ldsK, const float* ldsV, int n, const float4& q4, int grp,
                                           int dq, float& m, float& lsum, float4& o4) {
  // blocks of at most 32 rows (8 row groups) keep the registers of one block
  // small; a partial block uses 4 groups when it has at most 16 rows
  for (int b0 = 0; b0 < n; b0 += 32) {
    const int nb = min(32, n - b0);
    if (nb > 16) att_window_t<8>(ldsK + b0 * HD, ldsV + b0 * HD, nb, q4, grp, dq, m, lsum, o4);
    else att_window_t<4>(ldsK + b0 * HD, ldsV + b0 * HD, nb, q4, grp, dq, m, lsum, o4);
  }
}

// Row sums acc(lr) = sum_j part[lr*SPR + j] (ascending j).
template <class GEO, int D>
__device__ __forceinline__ float row_acc(const Smem<D>& sm, int lr) {
  float a = 0.f;
#pragma unroll
  for (int j = 0; j < GEO::SPR; ++j) a += sm.part[lr * GEO::SPR + j];
  return a;
}

// Poll NW tagged words src[idx[k]] (k < n) until their tags equal the step's
// epoch; out[k] = the words' values (0 for k >= n).
template <int NW>
__device__ __forceinline__ void poll_words(const u64* src, const int (&idx)[NW], int n, unsigned tag, float (&out)[NW],
                                           unsigned* err) {
  u64 w[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) w[k] = k < n ? tload(src + idx[k]) : ((u64)tag << 32);
  unsigned spins = 0;
  for (;;) {
    bool all = true;
#pragma unroll
    for (int k = 0; k < NW; ++k)
      if ((unsigned)(w[k] >> 32) != tag) all = false;
    if (all) break;
    if (++spins > SPIN_CAP || ((spins & 255u) == 0u && err_set(err))) {
      raise_err(err, 1u);
      break;
    }
#pragma unroll
    for (int k = 0; k < NW; ++k)
      if (k < n && (unsigned)(w[k] >> 32) != tag) w[k] = tload(src + idx[k]);
  }
#pragma unroll
  for (int k = 0; k < NW; ++k) out[k] = __uint_as_float((unsigned)w[k]);
}

// The glue waves (leader + helpers). Per GEMV phase each glue wave fetches a
// third of the phase's input into LDS and counts itself in in_ready; the GEMV
// waves start from that count, and the leader (which also needs the whole
// input: LayerNorm statistics, residuals) waits for the same count, then for
// the GEMV waves, and runs the epilogue. LayerNorm is folded into the GEMV
// (LayerPtrs::sq etc.): the GEMV input is x * g, and the leader's statistics
// are applied to the row sums in the epilogue, so they are computed while the
// GEMV waves run instead of before.
template <class C>
__device__ __forceinline__ void glue_role(const Params& p, Smem<C::D>& sm, int gw, int lane, int len, int NCH,
                                          int items, unsigned tag, uint32_t tok) {
  constexpr int D = C::D, H = C::H;
  typedef typename C::GQ GQ;
  typedef typename C::GP GP;
  typedef typename C::GF GF;
  typedef typename C::GM GM;
  typedef typename C::GL GL;
  const bool leader = gw == 0;
  const int gl = gw * 64 + lane;
  const int wg = blockIdx.x;
  unsigned gen = 0, seq = 0;
  const int pos = len - 1;
  // embedding (gpt2.rs:377-384): every workgroup computes x0 itself, each
  // glue wave a third of it
  if (leader) PK_TRACE(p, 0, lane);
  float c0q = 0.f;  // centre of the c_attn input (see LayerPtrs)
  {
    const float* g1 = PK_C(LayerPtrs, p.layers)[0].ln1w;
    for (int i = gl; i < D; i += NGLUE * 64) {
      float w;
      if (C::WT == W_F32) w = PK_G(float, p.wte)[(long)tok * D + i];
      else w = __uint_as_float((uint32_t)PK_G(uint16_t, p.wte)[(long)tok * D + i] << 16);
      sm.xraw[i] = w + PK_G(float, p.wpe)[(long)pos * D + i];
    }
    // layer 0's input centred on its own mean (no previous LayerNorm)
    glue_barrier(sm, gen, lane, p.err);
    c0q = lds_mean<D>(sm.xraw, lane);
    for (int i = gl; i < D; i += NGLUE * 64) sm.in_vec[1][i] = (sm.xraw[i] - c0q) * PK_G(float, g1)[i];
    glue_input_done(sm, PH_QKV, lane);
  }
  const int item = wg < items ? wg : -1;
  const int ih = item >= 0 ? item / NCH : 0, ic = item >= 0 ? item - ih * NCH : 0;
  const int CL = (len + NCH - 1) / NCH;
  const int j0 = ic * CL, j1 = min(len, j0 + CL);
  // Attention rows: the cached rows [j0, min(j1, pos)) of the item are split
  // between the NATT glue waves; the new row pos (when in the item) goes to
  // the last helper. Cached rows are final at step start, so each wave loads
  // its first window of a layer into LDS long before the layer's q is known.
  const int hw = gw;
  const int cend = min(j1, pos), per = (cend - j0 + NATT - 1) / NATT;
  const int h0 = min(cend, j0 + hw * per), h1 = min(cend, h0 + per);
  const bool has_new = hw == NATT - 1 && j1 == len;
  float* ldsK = sm.kv_k + hw * KVW * HD;
  float* ldsV = sm.kv_v + hw * KVW * HD;
  const long kv_head = (long)ih * p.P * HD;
  if (item >= 0 && h1 > h0)
    stage_rows(p.kc + kv_head, p.vc + kv_head, h0, min(KVW, h1 - h0), ldsK, ldsV, lane);
  for (int l = 0; l < p.L; ++l) {
    const __attribute__((address_space(4))) LayerPtrs& LP = PK_C(LayerPtrs, p.layers)[l];
    u64* T = p.tag + (long)l * p.lw;
    const int tb = 1 + 16 * l;  // trace index base of this layer
    float mean = 0.f, inv_std = 0.f;
    // ---- QKV: LN1(x) @ c_attn + bias; k/v of the new token into the cache ----
    {
      // the leader's epilogue constants, loaded before waiting for the input
      const int row0 = wg * GQ::RPW, rows_here = min(GQ::RPW, GQ::N - row0);
      float sr = 0.f, cr = 0.f;
      if (leader && lane < rows_here) {
        sr = PK_G(float, LP.sq)[row0 + lane];
        cr = PK_G(float, LP.cq)[row0 + lane];
      }
      if (l > 0) {  // centred on the mean of x2 of layer l - 1 (in LDS once all glue waves fetched it)
        const bool tw = p.test_spins != 0u && l == 1;  // the test hook's forced timeout
        glue_fetch<GM::RPW, GM::SW, D, true, D>(p.tag + (long)(l - 1) * p.lw + p.o_x3, D, tw ? tag + 0x5a5au : tag,
                                             sm.xraw, gl, p.err, sm.in_vec[1], LP.ln1w, sm.x2raw[(l - 1) & 1],
                                             &sm.in_ready[PH_FC], (unsigned)l * NGLUE, &c0q,
                                             tw ? p.test_spins : SPIN_CAP);
        glue_input_done(sm, PH_QKV, lane);
      }
      if (leader) {
        ++seq;
        lds_wait_ge(&sm.in_ready[PH_QKV], (unsigned)(l + 1) * NGLUE, p.err);
        PK_TRACE(p, tb + 0, lane);
        leader_ln_stats<D>(sm.xraw, p.eps, mean, inv_std, lane);
        PK_TRACE(p, 803 + 4 * l, lane);
        lds_wait_ge(&sm.gemv_done, seq * NC, p.err);
        PK_TRACE(p, tb + 1, lane);
        float* kl = p.kc + (long)l * p.kv_layer;
        float* vl = p.vc + (long)l * p.kv_layer;
        if (lane < rows_here) {
          const int n = row0 + lane;
          const float v = inv_std * (row_acc<GQ>(sm, lane) - (mean - c0q) * sr) + cr;
          tstore(T + p.o_qkv + wg * GQ::SW + lane, v, tag);
          if (n >= D) {
            const int c = n < 2 * D ? n - D : n - 2 * D;
            const int h = c / HD, dd = c - h * HD;
            float* base = n < 2 * D ? kl : vl;
            PK_GW(float, base)[((long)h * p.P + pos) * HD + dd] = v;
          }
        }
        PK_TRACE(p, tb + 2, lane);
      }
    }
    // ---- attention (multi_head_attention_cached, gpt2.rs:772-834): one item
    //      per workgroup = head ih, positions [j0, j1), on the glue waves ----
    if (item >= 0 && leader) {
      // q, k_new, v_new of head ih (one word per lane each), polled by the
      // leader and handed to the helpers through LDS
      float qkv[3];
      const int idx[3] = {slot_of<GQ::RPW, GQ::SW>(ih * HD + lane), slot_of<GQ::RPW, GQ::SW>(D + ih * HD + lane),
                          slot_of<GQ::RPW, GQ::SW>(2 * D + ih * HD + lane)};
      poll_words<3>(T + p.o_qkv, idx, 3, tag, qkv, p.err);
      sm.att_q[lane] = qkv[0];
      sm.att_k[lane] = qkv[1];
      sm.att_v[lane] = qkv[2];
      lds_release();
      if (lane == 0) lds_add(&sm.att_go, 1);
      PK_TRACE(p, tb + 3, lane);
    }
    if (item >= 0) {
      const int grp = lane >> 4, dq = (lane & 15) * 4;
      if (!leader) lds_wait_ge(&sm.att_go, (unsigned)(l + 1), p.err);
      if (gw == 1) PK_TRACE(p, 801 + 4 * l, lane);
      const float* Kh = p.kc + (long)l * p.kv_layer + kv_head;
      const float* Vh = p.vc + (long)l * p.kv_layer + kv_head;
      const float4 q4 = *reinterpret_cast<const float4*>(sm.att_q + dq);
      float m = -INFINITY, lsum = 0.f;
      float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int w0 = h0; w0 < h1; w0 += KVW) {
        const int n = min(KVW, h1 - w0);
        if (w0 > h0) stage_rows(Kh, Vh, w0, n, ldsK, ldsV, lane);  // windows after the first
        wait_vm_all();
        att_window(ldsK, ldsV, n, q4, grp, dq, m, lsum, o4);
      }
      if (has_new) {  // row pos: k/v of the new token, counted once (row group 0)
        const float4 k = *reinterpret_cast<const float4*>(sm.att_k + dq);
        const float4 v = *reinterpret_cast<const float4*>(sm.att_v + dq);
        const float s = row16_sum(q4.x * k.x + q4.y * k.y + q4.z * k.z + q4.w * k.w) * 0.125f;
        const float mn = fmaxf(m, s);
        const float corr = m == -INFINITY ? 0.f : fexp(m - mn);
        const float pj = grp == 0 ? fexp(s - mn) : 0.f;
        lsum = lsum * corr + pj;
        o4.x = o4.x * corr + pj * v.x;
        o4.y = o4.y * corr + pj * v.y;
        o4.z = o4.z * corr + pj * v.z;
        o4.w = o4.w * corr + pj * v.w;
        m = mn;
      }
      // sum over the 4 row groups
      lsum = xor32_sum(xor16_sum(lsum));
      o4.x = xor32_sum(xor16_sum(o4.x));
      o4.y = xor32_sum(xor16_sum(o4.y));
      o4.z = xor32_sum(xor16_sum(o4.z));
      o4.w = xor32_sum(xor16_sum(o4.w));
      if (lane < 16) {
        sm.att_part[hw][2 + dq + 0] = o4.x;
        sm.att_part[hw][2 + dq + 1] = o4.y;
        sm.att_part[hw][2 + dq + 2] = o4.z;
        sm.att_part[hw][2 + dq + 3] = o4.w;
      }
      if (lane == 0) {
        sm.att_part[hw][0] = m;  // -inf (and lsum 0) when this wave had no rows
        sm.att_part[hw][1] = lsum;
      }
      if (gw == 1) PK_TRACE(p, 802 + 4 * l, lane);
      // the wave that finishes last merges the waves' (m, l, o) into the
      // item's partial softmax and publishes it
      lds_release();
      unsigned arrived = 0;
      if (lane == 0) arrived = __hip_atomic_fetch_add(&sm.att_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      arrived = __builtin_amdgcn_readlane(arrived, 0);
      if (arrived == (unsigned)((l + 1) * NATT - 1)) {
        lds_acquire();
        PK_TRACE(p, tb + 4, lane);
        float M = -INFINITY;
        for (int w = 0; w < NATT; ++w) M = fmaxf(M, sm.att_part[w][0]);
        float Ls = 0.f, o = 0.f;
        for (int w = 0; w < NATT; ++w) {
          const float mw = sm.att_part[w][0];
          if (mw == -INFINITY) continue;
          const float f = fexp(mw - M);
          Ls += sm.att_part[w][1] * f;
          o += sm.att_part[w][2 + lane] * f;
        }
        // item slot: o[64], then m and l; a head in a single chunk publishes
        // its finished output o / l and the consumers use it as it is
        u64* dst = T + p.o_att + (long)item * ITEM_SLOT;
        if (NCH == 1) {
          tstore(dst + lane, o / Ls, tag);
        } else {
          tstore(dst + lane, o, tag);
          if (lane == 0) {
            tstore(dst + HD, M, tag);
            tstore(dst + HD + 1, Ls, tag);
          }
        }
      }
      if (l + 1 < p.L && h1 > h0) {  // the window is free again: load the next layer's first one
        const long nl = (long)(l + 1) * p.kv_layer + kv_head;
        stage_rows(p.kc + nl, p.vc + nl, h0, min(KVW, h1 - h0), ldsK, ldsV, lane);
      }
    }
    // ---- a head split into chunks: the workgroup holding its chunk 0 merges
    //      the chunks' partial softmaxes (m, l, o) and publishes o / l ----
    if (NCH > 1 && item >= 0 && ic == 0) {
      glue_fetch<ITEM_WORDS, ITEM_SLOT, CMAX * ITEM_WORDS>(T + p.o_att + (long)ih * NCH * ITEM_SLOT, NCH * ITEM_WORDS,
                                                          tag, sm.stage, gl, p.err);
      glue_barrier(sm, gen, lane, p.err);
      if (leader) {
        float M = -INFINITY;
        for (int c = 0; c < NCH; ++c) M = fmaxf(M, sm.stage[c * ITEM_WORDS + HD]);
        float Ls = 0.f, o = 0.f;
        for (int c = 0; c < NCH; ++c) {
          const float* it = sm.stage + c * ITEM_WORDS;
          if (it[HD] == -INFINITY) continue;
          const float f = fexp(it[HD] - M);
          Ls += it[HD + 1] * f;
          o += it[lane] * f;
        }
        tstore(T + p.o_head + (long)ih * ITEM_SLOT + lane, o / Ls, tag);
      }
    }
    // ---- attention projection + residual (gpt2.rs:523-526) ----
    {
      const int row0 = wg * GP::RPW, rows_here = min(GP::RPW, GP::N - row0);
      const float bias = leader && lane < rows_here ? PK_G(float, LP.baproj)[row0 + lane] : 0.f;
      // the heads' normalised outputs are the projection input: published by
      // the attention items themselves (one chunk per head) or by the mergers
      if (rows_here > 0)  // workgroups without projection rows count themselves in without the input
        glue_fetch<HD, ITEM_SLOT, H * HD>(T + (NCH == 1 ? p.o_att : p.o_head), H * HD, tag, sm.in_vec[0], gl,
                                          p.err);
      glue_input_done(sm, PH_PROJ, lane);
      if (leader) {
        PK_TRACE(p, tb + 5, lane);
        lds_wait_ge(&sm.gemv_done, ++seq * NC, p.err);
        PK_TRACE(p, tb + 6, lane);
        if (lane < rows_here)
          tstore(T + p.o_x2 + wg * GP::SW + lane, sm.xraw[row0 + lane] + (row_acc<GP>(sm, lane) + bias), tag);
        PK_TRACE(p, tb + 7, lane);
      }
    }
    // ---- FC + gelu_new (gpt2.rs:529-533), LN2 folded ----
    {
      const int row0 = wg * GF::RPW, rows_here = min(GF::RPW, GF::N - row0);
      float sr = 0.f, cr = 0.f;
      if (leader && lane < rows_here) {
        sr = PK_G(float, LP.sf)[row0 + lane];
        cr = PK_G(float, LP.cf)[row0 + lane];
      }
      // centred on the mean of this layer's input x (in LDS once all glue
      // waves delivered the c_attn input)
      float c0f = 0.f;
      glue_fetch<GP::RPW, GP::SW, D, true, D>(T + p.o_x2, D, tag, sm.x2raw[l & 1], gl, p.err, sm.in_vec[1],
                                              LP.ln2w, sm.xraw, &sm.in_ready[PH_QKV], (unsigned)(l + 1) * NGLUE,
                                              &c0f);
      glue_input_done(sm, PH_FC, lane);
      if (leader) {
        ++seq;
        lds_wait_ge(&sm.in_ready[PH_FC], (unsigned)(l + 1) * NGLUE, p.err);
        PK_TRACE(p, tb + 8, lane);
        leader_ln_stats<D>(sm.x2raw[l & 1], p.eps, mean, inv_std, lane);
        PK_TRACE(p, 800 + 4 * l, lane);
        lds_wait_ge(&sm.gemv_done, seq * NC, p.err);
        PK_TRACE(p, tb + 9, lane);
        if (lane < rows_here)
          tstore(T + p.o_h + wg * GF::SW + lane,
                 gelu_new(inv_std * (row_acc<GF>(sm, lane) - (mean - c0f) * sr) + cr), tag);
        PK_TRACE(p, tb + 10, lane);
      }
    }
    // ---- MLP projection + residual (gpt2.rs:534-537) ----
    {
      const int row0 = wg * GM::RPW, rows_here = min(GM::RPW, GM::N - row0);
      const float bias = leader && lane < rows_here ? PK_G(float, LP.bmproj)[row0 + lane] : 0.f;
      // all 4d words in one polling round up to d = 1024 (22 words per lane;
      // c3: 572.5 against 583 µs per token in two rounds of 3072); at the
      // larger widths, whose glue waves already spill registers, 3072 words
      // (16 per lane) per round
      glue_fetch<GF::RPW, GF::SW, (4 * D <= 4096 ? 4 * D : 3072)>(T + p.o_h, 4 * D, tag, sm.in_vec[0], gl, p.err);
      glue_input_done(sm, PH_MLP, lane);
      if (leader) {
        PK_TRACE(p, tb + 15, lane);
        lds_wait_ge(&sm.gemv_done, ++seq * NC, p.err);
        PK_TRACE(p, tb + 12, lane);
        if (lane < rows_here)
          tstore(T + p.o_x3 + wg * GM::SW + lane, sm.x2raw[l & 1][row0 + lane] + (row_acc<GM>(sm, lane) + bias),
                 tag);
        PK_TRACE(p, tb + 13, lane);
      }
    }
  }
  // ---- ln_f + tied LM head + argmax (gpt2.rs:392-396, 858-868), ln_f folded ----
  constexpr int NLR = (GL::RPW + 63) / 64;  // LM-head rows per leader lane
  const int row0 = wg * GL::RPW, rows_here = min(GL::RPW, p.V - row0);
  float sl[NLR], cl[NLR];
#pragma unroll
  for (int k = 0; k < NLR; ++k) {
    const int lr = lane + 64 * k;
    sl[k] = leader && lr < rows_here ? PK_G(float, p.sl)[row0 + lr] : 0.f;
    cl[k] = leader && lr < rows_here ? PK_G(float, p.cl)[row0 + lr] : 0.f;
  }
  float c0l = 0.f;
  glue_fetch<GM::RPW, GM::SW, D, true, D>(p.tag + (long)(p.L - 1) * p.lw + p.o_x3, D, tag, sm.xraw, gl, p.err,
                                       sm.in_vec[1], p.lnfw, sm.x2raw[(p.L - 1) & 1], &sm.in_ready[PH_FC],
                                       (unsigned)p.L * NGLUE, &c0l);
  glue_input_done(sm, PH_LM, lane);
  if (leader) {
    ++seq;
    lds_wait_ge(&sm.in_ready[PH_LM], NGLUE, p.err);
    PK_TRACE(p, 1 + 16 * p.L, lane);
    float mean, inv_std;
    leader_ln_stats<D>(sm.xraw, p.eps, mean, inv_std, lane);
    lds_wait_ge(&sm.gemv_done, seq * NC, p.err);
    PK_TRACE(p, 2 + 16 * p.L, lane);
    u64 best = 0ull;
#pragma unroll
    for (int k = 0; k < NLR; ++k) {
      const int lr = lane + 64 * k;
      if (lr < rows_here) {
        const int n = row0 + lr;
        const float v = inv_std * (row_acc<GL>(sm, lr) - (mean - c0l) * sl[k]) + cl[k];
        PK_GW(float, p.logits)[n] = v;
        const u64 key = argmax_key(v, (uint32_t)n);  // -inf and NaN give 0: they never win
        best = key > best ? key : best;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const u64 other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    u64 prev = 0ull;
    if (lane == 0 && best != 0ull)
      prev = __hip_atomic_fetch_max(PK_GW(u64, p.keys), best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    PK_TRACE(p, 3 + 16 * p.L, lane);
    // The last workgroup to arrive finishes the step (finalize of the
    // reference loop, gpt2.rs:431-437: push the argmax token, feed it back):
    // each workgroup's key update has completed (s_waitcnt) before it counts
    // itself, so the last arrival reads the final key.
    if (lane == 0) {
      asm volatile("" : : "v"(prev));      // the returned value: the atomic max has been performed
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
      const unsigned arrived = __hip_atomic_fetch_add(PK_GW(unsigned, p.done), 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
      if (arrived == G - 1) {
        const u64 key = __hip_atomic_load(PK_GW(u64, p.keys), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t next = argmax_key_index(key);
        const int step = *PK_G(int, p.step);
        PK_GW(uint32_t, p.token)[0] = next;
        PK_GW(uint32_t, p.ids_out)[step] = next;
        PK_GW(u64, p.keys)[0] = 0ull;
        PK_GW(int, p.pos)[0] = pos + 1;
        PK_GW(int, p.step)[0] = step + 1;
        PK_GW(unsigned, p.epoch)[0] = tag + 1u;
        PK_GW(unsigned, p.done)[0] = 0u;
      }
    }
  }
}

// Attention chunking for this step: NCH chunks per head, one per KVS
// positions (so each chunk fits the LDS stage and each attention wave holds
// one window, loaded a layer ahead), at most CMAX and H*NCH <= G. Every
// workgroup then reads only the H merged head outputs.
template <int H>
__device__ __host__ __forceinline__ int att_chunks(int len) {
  constexpr int cap0 = CMAX < MAX_ITEMS / H ? CMAX : MAX_ITEMS / H;
  constexpr int cap = cap0 < G / H ? cap0 : G / H;
  int c = (len + KVS - 1) / KVS;
  c = c < cap ? c : cap;
  return c < 1 ? 1 : c;
}

template <int D, int V, int WT>
__global__ __launch_bounds__(NTHREADS) void decode_step_kernel(Params p) {
  typedef Cfg<D, V, WT> C;
  __shared__ Smem<D> sm;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (threadIdx.x == 0) {
    for (int i = 0; i < 5; ++i) sm.in_ready[i] = 0;
    sm.att_go = 0;
    sm.att_cnt = 0;
    sm.gemv_done = 0;
    sm.glue_cnt = 0;
    sm.trace_t0 = wall_clock64();
  }
  if (p.trace)
    for (int i = threadIdx.x; i < TRACE_N; i += NTHREADS) sm.trace_rel[i] = 0;
  __syncthreads();
  // step inputs, loaded together (written by the previous step's last workgroup)
  const int len = *PK_G(int, p.pos) + 1;
  const unsigned tag = *PK_G(unsigned, p.epoch);
  const uint32_t tok = *PK_G(uint32_t, p.token);
  const int nch = att_chunks<C::H>(len);
  if (wave < NGLUE) glue_role<C>(p, sm, wave, lane, len, nch, C::H * nch, tag, tok);
  else gemv_role<C>(p, sm, wave - NGLUE, lane);
  if (p.trace) {
    __syncthreads();
    for (int i = threadIdx.x; i < TRACE_N; i += NTHREADS) {
      const unsigned r = sm.trace_rel[i];
      PK_GW(u64, p.trace)[(long)blockIdx.x * TRACE_STRIDE + i] = r ? sm.trace_t0 + r : 0ull;
    }
  }
}

}  // namespace pk
}  // namespace rtg
