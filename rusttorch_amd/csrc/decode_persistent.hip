// Persistent decode step for batch 1: one cooperative launch runs a whole
// forward_cached(&[token]) + argmax (gpt2.rs:358-399, 858-868) across all CUs.
//
// Design (MI355X, 256 CUs, one workgroup per CU):
//  * Every weight matrix is streamed exactly once per step. Each workgroup
//    owns a contiguous block of output rows of every phase; its GEMV waves
//    hold their share of a phase's weights in registers, loaded one phase
//    ahead (two register buffers A/B), so HBM keeps streaming while the
//    workgroups exchange activations.
//  * Workgroups exchange activations without grid barriers or agent-scope
//    fences (each of those costs ~1-2 us here): every published value is a
//    64-bit word {tag, f32} written with one relaxed agent-scope atomic
//    store, and consumers poll the words they need until every tag equals
//    the step's epoch. Each (layer, phase) has its own buffer, so a word is
//    written once per step and never overwritten while someone may read it.
//  * Waves are specialised so that no wave that owns in-flight prefetch
//    loads ever waits on vmcnt(0) for a publication:
//      wave 0            leader: LayerNorm, attention merge, epilogues, stores
//      waves 1..NA       helpers: poll inputs with the leader, attention
//      waves NA+1..      GEMV waves: weights in registers, dot products
//    Leader/helpers and GEMV waves meet only through LDS counters.
//  * Every wait is bounded; a timeout sets *err and lets the step finish
//    (with wrong numbers) instead of hanging; the host reports the error.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "decode_persistent.h"
#include "kernels.h"

namespace rtg {
namespace {

constexpr int NA = 3;                    // helper waves
constexpr int NC = 8;                    // GEMV waves
constexpr int NGLUE = 1 + NA;            // leader + helpers
constexpr int NTHREADS = (1 + NA + NC) * 64;
constexpr int HD = 64;                   // head_dim (all GPT-2 sizes)
constexpr int CMAX = 16;                 // attention chunks per head
constexpr int ITEM_WORDS = 2 + HD;       // m, l, o[64]
constexpr int MAX_ITEMS = 64;            // heads * chunks handled by consumer-side merge
constexpr int MAXW = 12;                 // polled words per glue lane per round
constexpr int DMAX = 1600;
constexpr int PART_MAX = 1024;           // segment partials per workgroup
constexpr int ATT_POS_MAX = 256;         // positions per helper wave per item
constexpr unsigned SPIN_CAP = 1u << 21;

typedef unsigned long long u64;

struct Geom {
  int N, K, VR, spr, rows_per_wg, spw;  // spw: segments per GEMV wave
};

struct LayerPtrs {
  const void *wqkv, *waproj, *wfc, *wmproj;
  const float *bqkv, *baproj, *bfc, *bmproj, *ln1w, *ln1b, *ln2w, *ln2b;
};

struct Params {
  const LayerPtrs* layers;
  const void* wte;
  const float *wpe, *lnfw, *lnfb;
  int L, d, H, V, P, wtype;
  float eps;
  Geom gq, gp, gf, gm, glm;
  float* kc;  // [L][H][P][HD]
  float* vc;
  long kv_layer;  // floats per layer
  const uint32_t* token;
  const int* pos;
  const unsigned* epoch;
  u64* tag;  // tagged words, lw per layer
  long lw;
  int o_qkv, o_att, o_x2, o_h, o_x3;
  float* logits;
  u64* keys;
  unsigned* err;
};

struct Smem {
  float in_vec[2][4 * DMAX];  // GEMV input, double-buffered by phase parity
  float xraw[DMAX];   // residual input of the current layer
  float x2raw[DMAX];  // residual after attention
  float part[PART_MAX];
  float stage[MAX_ITEMS * ITEM_WORDS];
  float att_q[HD], att_k[HD], att_v[HD];
  float att_s[NA][ATT_POS_MAX];
  float att_part[NA][ITEM_WORDS];
  float red[8];
  unsigned gemv_ready, gemv_done, glue_cnt;
};

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ u64 tload(const u64* p) {
  return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(u64* p, float v, unsigned tag) {
  __hip_atomic_store(p, ((u64)tag << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned lds_load(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(unsigned* p, unsigned v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Order this wave's LDS accesses (lgkmcnt only; never waits on vmcnt).
__device__ __forceinline__ void lds_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local"); }
__device__ __forceinline__ void lds_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local"); }

__device__ __forceinline__ bool err_set(const unsigned* err) {
  return __hip_atomic_load(const_cast<unsigned*>(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void raise_err(unsigned* err, unsigned code) {
  __hip_atomic_fetch_or(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float gelu_new(float x) {
  const float sqrt_2_pi = 0.7978845608028654f;
  float inner = sqrt_2_pi * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

template <int WT>
struct V16;
template <>
struct V16<W_F32> {
  typedef float4 T;
  static constexpr int E = 4;
  __device__ __forceinline__ static T load(const void* b, long i) { return reinterpret_cast<const float4*>(b)[i]; }
  __device__ __forceinline__ static float dot(const T& w, const float* x) {
    const float4 xv = *reinterpret_cast<const float4*>(x);
    return w.x * xv.x + w.y * xv.y + w.z * xv.z + w.w * xv.w;
  }
};
template <>
struct V16<W_BF16> {
  typedef uint4 T;
  static constexpr int E = 8;
  __device__ __forceinline__ static T load(const void* b, long i) { return reinterpret_cast<const uint4*>(b)[i]; }
  __device__ __forceinline__ static float dot(const T& w, const float* x) {
    const float4 a = *reinterpret_cast<const float4*>(x);
    const float4 c = *reinterpret_cast<const float4*>(x + 4);
    float s = __uint_as_float(w.x << 16) * a.x + __uint_as_float(w.x & 0xffff0000u) * a.y;
    s += __uint_as_float(w.y << 16) * a.z + __uint_as_float(w.y & 0xffff0000u) * a.w;
    s += __uint_as_float(w.z << 16) * c.x + __uint_as_float(w.z & 0xffff0000u) * c.y;
    s += __uint_as_float(w.w << 16) * c.z + __uint_as_float(w.w & 0xffff0000u) * c.w;
    return s;
  }
};

// ---------------------------------------------------------------------------
// GEMV waves: segment s of a workgroup = 64 consecutive 16-byte vectors of
// one output row (the last segment of a row may be partial).
// ---------------------------------------------------------------------------

template <int WT, int MAXSEG>
__device__ __forceinline__ void seg_issue(typename V16<WT>::T (&buf)[MAXSEG], const void* W, const Geom& g, int wg,
                                          int cw, int lane, int seg_base) {
  const int row0 = wg * g.rows_per_wg;
  const int rows_here = min(g.rows_per_wg, g.N - row0);
  const int segs_here = rows_here > 0 ? rows_here * g.spr : 0;
  int s = seg_base + cw * g.spw;
  int lr = s / g.spr, j = s - lr * g.spr;
  const int s_end = min(seg_base + (cw + 1) * g.spw, segs_here);
#pragma unroll
  for (int i = 0; i < MAXSEG; ++i) {
    if (s < s_end) {
      const int v = j * 64 + lane;
      if (v < g.VR) buf[i] = V16<WT>::load(W, (long)(row0 + lr) * g.VR + v);
    }
    ++s;
    if (++j == g.spr) {
      j = 0;
      ++lr;
    }
  }
}

template <int WT, int MAXSEG>
__device__ __forceinline__ void seg_compute(const typename V16<WT>::T (&buf)[MAXSEG], const float* x, float* part,
                                            const Geom& g, int wg, int cw, int lane, int seg_base, int part_base) {
  constexpr int E = V16<WT>::E;
  const int row0 = wg * g.rows_per_wg;
  const int rows_here = min(g.rows_per_wg, g.N - row0);
  const int segs_here = rows_here > 0 ? rows_here * g.spr : 0;
  int s = seg_base + cw * g.spw;
  int j = s % g.spr;
  const int s_end = min(seg_base + (cw + 1) * g.spw, segs_here);
#pragma unroll
  for (int i = 0; i < MAXSEG; ++i) {
    if (s < s_end) {
      const int v = j * 64 + lane;
      float acc = 0.f;
      if (v < g.VR) acc = V16<WT>::dot(buf[i], x + v * E);
      acc = wsum(acc);
      if (lane == 0) part[s - part_base] = acc;
    }
    ++s;
    if (++j == g.spr) j = 0;
  }
}

template <int WT, int MAXSEG>
__device__ void gemv_role(const Params& p, Smem& sm, int cw, int lane) {
  typedef typename V16<WT>::T Vec;
  const int wg = blockIdx.x;
  Vec A[MAXSEG], B[MAXSEG];
  unsigned seq = 0;
  const LayerPtrs* LP = p.layers;
  // Prologue: first two weight phases of layer 0.
  seg_issue<WT, MAXSEG>(A, LP[0].wqkv, p.gq, wg, cw, lane, 0);
  seg_issue<WT, MAXSEG>(B, LP[0].waproj, p.gp, wg, cw, lane, 0);
  for (int l = 0; l < p.L; ++l) {
    const LayerPtrs& cur = LP[l];
    const bool last = l + 1 == p.L;
    // QKV (A), then prefetch FC into A
    lds_wait_ge(&sm.gemv_ready, ++seq, p.err);
    seg_compute<WT, MAXSEG>(A, sm.in_vec[1], sm.part, p.gq, wg, cw, lane, 0, 0);
    lds_release();
    if (lane == 0) lds_add(&sm.gemv_done, 1);
    seg_issue<WT, MAXSEG>(A, cur.wfc, p.gf, wg, cw, lane, 0);
    // attention projection (B), then prefetch the MLP projection into B
    lds_wait_ge(&sm.gemv_ready, ++seq, p.err);
    seg_compute<WT, MAXSEG>(B, sm.in_vec[0], sm.part, p.gp, wg, cw, lane, 0, 0);
    lds_release();
    if (lane == 0) lds_add(&sm.gemv_done, 1);
    seg_issue<WT, MAXSEG>(B, cur.wmproj, p.gm, wg, cw, lane, 0);
    // FC (A), then prefetch next layer's QKV (or the LM head's first chunk)
    lds_wait_ge(&sm.gemv_ready, ++seq, p.err);
    seg_compute<WT, MAXSEG>(A, sm.in_vec[1], sm.part, p.gf, wg, cw, lane, 0, 0);
    lds_release();
    if (lane == 0) lds_add(&sm.gemv_done, 1);
    if (!last) seg_issue<WT, MAXSEG>(A, LP[l + 1].wqkv, p.gq, wg, cw, lane, 0);
    else seg_issue<WT, MAXSEG>(A, p.wte, p.glm, wg, cw, lane, 0);
    // MLP projection (B), then prefetch next layer's attention projection
    lds_wait_ge(&sm.gemv_ready, ++seq, p.err);
    seg_compute<WT, MAXSEG>(B, sm.in_vec[0], sm.part, p.gm, wg, cw, lane, 0, 0);
    lds_release();
    if (lane == 0) lds_add(&sm.gemv_done, 1);
    if (!last) seg_issue<WT, MAXSEG>(B, LP[l + 1].waproj, p.gp, wg, cw, lane, 0);
    else seg_issue<WT, MAXSEG>(B, p.wte, p.glm, wg, cw, lane, NC * p.glm.spw);
  }
  // LM head: the wave's segments come in chunks of spw; chunk c covers
  // workgroup segments [c * NC * spw, (c + 1) * NC * spw).
  lds_wait_ge(&sm.gemv_ready, ++seq, p.err);
  const int row0 = wg * p.glm.rows_per_wg;
  const int rows_here = min(p.glm.rows_per_wg, p.glm.N - row0);
  const int segs_here = rows_here > 0 ? rows_here * p.glm.spr : 0;
  const int per_chunk = NC * p.glm.spw;
  for (int base = 0; base < segs_here; base += 2 * per_chunk) {
    seg_compute<WT, MAXSEG>(A, sm.in_vec[1], sm.part, p.glm, wg, cw, lane, base, 0);
    if (base + 2 * per_chunk < segs_here) seg_issue<WT, MAXSEG>(A, p.wte, p.glm, wg, cw, lane, base + 2 * per_chunk);
    if (base + per_chunk < segs_here) {
      seg_compute<WT, MAXSEG>(B, sm.in_vec[1], sm.part, p.glm, wg, cw, lane, base + per_chunk, 0);
      if (base + 3 * per_chunk < segs_here)
        seg_issue<WT, MAXSEG>(B, p.wte, p.glm, wg, cw, lane, base + 3 * per_chunk);
    }
  }
  lds_release();
  if (lane == 0) lds_add(&sm.gemv_done, 1);
}

// ---------------------------------------------------------------------------
// Leader + helper waves ("glue").
// ---------------------------------------------------------------------------

// Barrier among the NGLUE glue waves (monotonic LDS counter).
__device__ __forceinline__ void glue_barrier(Smem& sm, unsigned& gen, int lane, unsigned* err) {
  ++gen;
  lds_release();
  if (lane == 0) lds_add(&sm.glue_cnt, 1);
  lds_wait_ge(&sm.glue_cnt, gen * NGLUE, err);
}

// All glue lanes (gl in [0, NGLUE*64)) poll n tagged words into dst, in
// rounds of MAXW words per lane (all loads of a round in flight at once).
__device__ void glue_poll(const u64* src, int n, unsigned tag, float* dst, int gl, unsigned* err) {
  constexpr int NG = NGLUE * 64;
  const bool skip = err_set(err);
  for (int base = 0; base < n; base += MAXW * NG) {
    u64 w[MAXW];
#pragma unroll
    for (int k = 0; k < MAXW; ++k) {
      const int i = base + gl + k * NG;
      w[k] = (i < n && !skip) ? tload(src + i) : ((u64)tag << 32);
    }
    unsigned spins = 0;
    for (;;) {
      bool all = true;
#pragma unroll
      for (int k = 0; k < MAXW; ++k)
        if ((unsigned)(w[k] >> 32) != tag) all = false;
      if (all) break;
      if (++spins > SPIN_CAP || ((spins & 255u) == 0u && err_set(err))) {
        raise_err(err, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
#pragma unroll
      for (int k = 0; k < MAXW; ++k) {
        const int i = base + gl + k * NG;
        if (i < n && (unsigned)(w[k] >> 32) != tag) w[k] = tload(src + i);
      }
    }
#pragma unroll
    for (int k = 0; k < MAXW; ++k) {
      const int i = base + gl + k * NG;
      if (i < n) dst[i] = __uint_as_float((unsigned)w[k]);
    }
  }
}

// Leader only: LayerNorm of src[d] into dst (gpt2.rs:636-666, two-pass).
__device__ void leader_layernorm(const float* src, const float* w, const float* b, float eps, int d, float* dst,
                                 int lane) {
  float s = 0.f;
  for (int i = lane; i < d; i += 64) s += src[i];
  const float mean = wsum(s) / (float)d;
  float v = 0.f;
  for (int i = lane; i < d; i += 64) {
    const float t = src[i] - mean;
    v += t * t;
  }
  const float var = wsum(v) / (float)d;
  const float inv_std = 1.0f / sqrtf(var + eps);
  for (int i = lane; i < d; i += 64) dst[i] = (src[i] - mean) * inv_std * w[i] + b[i];
}

// Leader only: publish in_vec to the GEMV waves and wait for their partials.
__device__ __forceinline__ void leader_run_gemv(Smem& sm, unsigned& seq, int lane, unsigned* err) {
  lds_release();
  ++seq;
  if (lane == 0) __hip_atomic_store(&sm.gemv_ready, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  lds_wait_ge(&sm.gemv_done, seq * NC, err);
}

// Leader only: row sums of the workgroup's rows: acc(lr) = sum_j part[lr*spr + j].
__device__ __forceinline__ float row_acc(const Smem& sm, const Geom& g, int lr) {
  float a = 0.f;
  for (int j = 0; j < g.spr; ++j) a += sm.part[lr * g.spr + j];
  return a;
}

__device__ void glue_role(const Params& p, Smem& sm, int gw, int lane, int len, int C, int items, unsigned tag) {
  const bool leader = gw == 0;
  const int gl = gw * 64 + lane;
  const int wg = blockIdx.x;
  const int d = p.d, H = p.H;
  unsigned gen = 0, seq = 0;
  const int pos = len - 1;
  // embedding (gpt2.rs:377-384): every workgroup computes x0 itself
  if (leader) {
    const uint32_t tok = *p.token;
    for (int i = lane; i < d; i += 64) {
      float w;
      if (p.wtype == W_F32) w = reinterpret_cast<const float*>(p.wte)[(long)tok * d + i];
      else w = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p.wte)[(long)tok * d + i] << 16);
      sm.xraw[i] = w + p.wpe[(long)pos * d + i];
    }
  }
  const int item = wg < items ? wg : -1;
  const int ih = item >= 0 ? item / C : 0, ic = item >= 0 ? item - (item / C) * C : 0;
  const int CL = (len + C - 1) / C;
  const int j0 = ic * CL, j1 = min(len, j0 + CL);
  for (int l = 0; l < p.L; ++l) {
    const LayerPtrs& LP = p.layers[l];
    u64* T = p.tag + (long)l * p.lw;
    // ---- QKV ----
    if (l > 0) {
      glue_poll(p.tag + (long)(l - 1) * p.lw + p.o_x3, d, tag, sm.xraw, gl, p.err);
      glue_barrier(sm, gen, lane, p.err);
    }
    if (leader) {
      leader_layernorm(sm.xraw, LP.ln1w, LP.ln1b, p.eps, d, sm.in_vec[1], lane);
      leader_run_gemv(sm, seq, lane, p.err);
      const Geom& g = p.gq;
      const int row0 = wg * g.rows_per_wg, rows_here = min(g.rows_per_wg, g.N - row0);
      float* kl = p.kc + (long)l * p.kv_layer;
      float* vl = p.vc + (long)l * p.kv_layer;
      for (int lr = lane; lr < rows_here; lr += 64) {
        const int n = row0 + lr;
        const float v = row_acc(sm, g, lr) + LP.bqkv[n];
        tstore(T + p.o_qkv + n, v, tag);
        if (n >= d) {
          const int c = n < 2 * d ? n - d : n - 2 * d;
          const int h = c / HD, dd = c - h * HD;
          float* base = n < 2 * d ? kl : vl;
          base[((long)h * p.P + pos) * HD + dd] = v;
        }
      }
    }
    // ---- attention (one item per workgroup: head ih, positions [j0, j1)) ----
    if (item >= 0) {
      if (leader) {
        float* dsts[3] = {sm.att_q, sm.att_k, sm.att_v};
        // q, k_new, v_new of head ih: 3 x 64 words
        for (int part = 0; part < 3; ++part) {
          const u64* src = T + p.o_qkv + part * d + ih * HD;
          u64 w = tload(src + lane);
          unsigned spins = 0;
          while ((unsigned)(w >> 32) != tag) {
            if (++spins > SPIN_CAP || ((spins & 255u) == 0u && err_set(p.err))) {
              raise_err(p.err, 1u);
              break;
            }
            __builtin_amdgcn_s_sleep(2);
            w = tload(src + lane);
          }
          dsts[part][lane] = __uint_as_float((unsigned)w);
        }
      }
      glue_barrier(sm, gen, lane, p.err);
      if (!leader) {
        // helper hw handles positions [a0, a1) of the item
        const int hw = gw - 1;
        const int per = (j1 - j0 + NA - 1) / NA;
        const int a0 = j0 + hw * per, a1 = min(j1, a0 + per);
        const float* Kh = p.kc + (long)l * p.kv_layer + (long)ih * p.P * HD;
        const float* Vh = p.vc + (long)l * p.kv_layer + (long)ih * p.P * HD;
        const int grp = lane >> 4, dq = (lane & 15) * 4;
        const float scale = 0.125f;  // 1 / sqrt(64)
        const float4 q4 = *reinterpret_cast<const float4*>(sm.att_q + dq);
        float mloc = -INFINITY;
        for (int jb = a0; jb < a1; jb += 4) {  // 4 positions per iteration, 16 lanes each
          const int j = jb + grp;
          float s = -INFINITY;
          float dot = 0.f;
          if (j < a1) {
            const float4 k4 = j == pos ? *reinterpret_cast<const float4*>(sm.att_k + dq)
                                       : *reinterpret_cast<const float4*>(Kh + (long)j * HD + dq);
            dot = q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
          }
#pragma unroll
          for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 64);
          if (j < a1) {
            s = dot * scale;
            if ((lane & 15) == 0) sm.att_s[hw][j - a0] = s;
          }
          mloc = fmaxf(mloc, s);
        }
        const float m = wmax(mloc);
        lds_release();
        lds_acquire();
        float lsum = 0.f;
        float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int jb = a0; jb < a1; jb += 4) {
          const int j = jb + grp;
          if (j >= a1) continue;
          const float pj = expf(sm.att_s[hw][j - a0] - m);
          const float4 v4 = j == pos ? *reinterpret_cast<const float4*>(sm.att_v + dq)
                                     : *reinterpret_cast<const float4*>(Vh + (long)j * HD + dq);
          if ((lane & 15) == 0) lsum += pj;
          o4.x += pj * v4.x;
          o4.y += pj * v4.y;
          o4.z += pj * v4.z;
          o4.w += pj * v4.w;
        }
        lsum = wsum(lsum);
#pragma unroll
        for (int o = 16; o < 64; o <<= 1) {
          o4.x += __shfl_xor(o4.x, o, 64);
          o4.y += __shfl_xor(o4.y, o, 64);
          o4.z += __shfl_xor(o4.z, o, 64);
          o4.w += __shfl_xor(o4.w, o, 64);
        }
        if (lane < 16) {
          sm.att_part[hw][2 + dq + 0] = o4.x;
          sm.att_part[hw][2 + dq + 1] = o4.y;
          sm.att_part[hw][2 + dq + 2] = o4.z;
          sm.att_part[hw][2 + dq + 3] = o4.w;
        }
        if (lane == 0) {
          sm.att_part[hw][0] = a1 > a0 ? m : -INFINITY;
          sm.att_part[hw][1] = a1 > a0 ? lsum : 0.f;
        }
      }
      glue_barrier(sm, gen, lane, p.err);
      if (leader) {
        float M = -INFINITY;
        for (int w = 0; w < NA; ++w) M = fmaxf(M, sm.att_part[w][0]);
        float Ls = 0.f, o = 0.f;
        for (int w = 0; w < NA; ++w) {
          const float mw = sm.att_part[w][0];
          if (mw == -INFINITY) continue;
          const float f = expf(mw - M);
          Ls += sm.att_part[w][1] * f;
          o += sm.att_part[w][2 + lane] * f;
        }
        u64* dst = T + p.o_att + (long)item * ITEM_WORDS;
        tstore(dst + 2 + lane, o, tag);
        if (lane == 0) {
          tstore(dst, M, tag);
          tstore(dst + 1, Ls, tag);
        }
      }
    }
    // ---- attention projection + residual ----
    glue_poll(T + p.o_att, items * ITEM_WORDS, tag, sm.stage, gl, p.err);
    glue_barrier(sm, gen, lane, p.err);
    if (leader) {
      for (int h = 0; h < H; ++h) {
        float M = -INFINITY;
        for (int c = 0; c < C; ++c) M = fmaxf(M, sm.stage[(h * C + c) * ITEM_WORDS]);
        float Ls = 0.f, o = 0.f;
        for (int c = 0; c < C; ++c) {
          const float* it = sm.stage + (h * C + c) * ITEM_WORDS;
          if (it[0] == -INFINITY) continue;
          const float f = expf(it[0] - M);
          Ls += it[1] * f;
          o += it[2 + lane] * f;
        }
        sm.in_vec[0][h * HD + lane] = o / Ls;
      }
      leader_run_gemv(sm, seq, lane, p.err);
      const Geom& g = p.gp;
      const int row0 = wg * g.rows_per_wg, rows_here = min(g.rows_per_wg, g.N - row0);
      for (int lr = lane; lr < rows_here; lr += 64) {
        const int n = row0 + lr;
        tstore(T + p.o_x2 + n, sm.xraw[n] + (row_acc(sm, g, lr) + LP.baproj[n]), tag);
      }
    }
    // ---- FC + GELU ----
    glue_poll(T + p.o_x2, d, tag, sm.x2raw, gl, p.err);
    glue_barrier(sm, gen, lane, p.err);
    if (leader) {
      leader_layernorm(sm.x2raw, LP.ln2w, LP.ln2b, p.eps, d, sm.in_vec[1], lane);
      leader_run_gemv(sm, seq, lane, p.err);
      const Geom& g = p.gf;
      const int row0 = wg * g.rows_per_wg, rows_here = min(g.rows_per_wg, g.N - row0);
      for (int lr = lane; lr < rows_here; lr += 64) {
        const int n = row0 + lr;
        tstore(T + p.o_h + n, gelu_new(row_acc(sm, g, lr) + LP.bfc[n]), tag);
      }
    }
    // ---- MLP projection + residual ----
    glue_poll(T + p.o_h, 4 * d, tag, sm.in_vec[0], gl, p.err);
    glue_barrier(sm, gen, lane, p.err);
    if (leader) {
      leader_run_gemv(sm, seq, lane, p.err);
      const Geom& g = p.gm;
      const int row0 = wg * g.rows_per_wg, rows_here = min(g.rows_per_wg, g.N - row0);
      for (int lr = lane; lr < rows_here; lr += 64) {
        const int n = row0 + lr;
        tstore(T + p.o_x3 + n, sm.x2raw[n] + (row_acc(sm, g, lr) + LP.bmproj[n]), tag);
      }
    }
  }
  // ---- ln_f + LM head + argmax ----
  glue_poll(p.tag + (long)(p.L - 1) * p.lw + p.o_x3, d, tag, sm.xraw, gl, p.err);
  glue_barrier(sm, gen, lane, p.err);
  if (leader) {
    leader_layernorm(sm.xraw, p.lnfw, p.lnfb, p.eps, d, sm.in_vec[1], lane);
    leader_run_gemv(sm, seq, lane, p.err);
    const Geom& g = p.glm;
    const int row0 = wg * g.rows_per_wg, rows_here = min(g.rows_per_wg, g.N - row0);
    u64 best = 0ull;
    for (int lr = lane; lr < rows_here; lr += 64) {
      const int n = row0 + lr;
      const float v = row_acc(sm, g, lr);
      p.logits[n] = v;
      u64 k = 0ull;
      if (v > -INFINITY) {  // -inf and NaN never win (strict '>' from -inf)
        uint32_t b = __float_as_uint(v);
        b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
        k = ((u64)b << 32) | (u64)(~(uint32_t)n);
      }
      best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const u64 other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if (lane == 0 && best != 0ull)
      __hip_atomic_fetch_max(p.keys, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int WT, int MAXSEG>
__global__ __launch_bounds__(NTHREADS) void decode_step_kernel(Params p) {
  __shared__ Smem sm;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (threadIdx.x == 0) {
    sm.gemv_ready = 0;
    sm.gemv_done = 0;
    sm.glue_cnt = 0;
  }
  __syncthreads();
  const int len = *p.pos + 1;
  const unsigned tag = *p.epoch;
  int C = (len + 31) / 32;
  const int cap = min(CMAX, min(MAX_ITEMS / p.H, (int)gridDim.x / p.H));
  C = max(1, min(C, cap));
  if ((len + C - 1) / C > NA * ATT_POS_MAX) C = cap;  // keep per-wave positions bounded
  const int items = p.H * C;
  if (wave < NGLUE) glue_role(p, sm, wave, lane, len, C, items, tag);
  else gemv_role<WT, MAXSEG>(p, sm, wave - NGLUE, lane);
}

Geom make_geom(int N, int K, int E, int G) {
  Geom g;
  g.N = N;
  g.K = K;
  g.VR = K / E;
  g.spr = (g.VR + 63) / 64;
  g.rows_per_wg = (N + G - 1) / G;
  const int segs = g.rows_per_wg * g.spr;
  g.spw = (segs + NC - 1) / NC;
  return g;
}

}  // namespace

struct PersistentPlan {
  PersistentWeights w;
  int G = 0;
  int maxseg = 0;  // 0: unsupported
  Params base{};
  LayerPtrs* layers_dev = nullptr;
};

struct PersistentState {
  PersistentPlan* plan;
  Params p;
  u64* tags = nullptr;
  unsigned* epoch = nullptr;
  unsigned* err = nullptr;
};

PersistentPlan* persistent_plan_create(const PersistentWeights& w) {
  PersistentPlan* pl = new PersistentPlan();
  pl->w = w;
  const int d = (int)w.cfg.n_embd, H = (int)w.cfg.n_head, V = (int)w.cfg.vocab_size, L = (int)w.cfg.n_layer;
  int dev = 0, cus = 0;
  hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return pl;
  const int E = w.wtype == W_BF16 ? 8 : 4;
  if (H <= 0 || d != H * HD || d > DMAX || L <= 0 || H > MAX_ITEMS || d % 8 != 0) return pl;
  const int G = cus;
  Params& p = pl->base;
  p.gq = make_geom(3 * d, d, E, G);
  p.gp = make_geom(d, d, E, G);
  p.gf = make_geom(4 * d, d, E, G);
  p.gm = make_geom(d, 4 * d, E, G);
  p.glm = make_geom(V, d, E, G);
  const int maxspw = std::max({p.gq.spw, p.gp.spw, p.gf.spw, p.gm.spw});
  const int lm_segs = p.glm.rows_per_wg * p.glm.spr;
  for (const Geom* g : {&p.gq, &p.gp, &p.gf, &p.gm})
    if (g->rows_per_wg * g->spr > PART_MAX) return pl;
  if (lm_segs > PART_MAX) return pl;
  int maxseg = maxspw <= 8 ? 8 : (maxspw <= 16 ? 16 : 0);
  if (!maxseg) return pl;
  // the LM head streams in chunks of spw; give it the same chunk size
  p.glm.spw = maxseg;
  std::vector<LayerPtrs> lp(L);
  for (int i = 0; i < L; ++i) {
    const PersistentLayer& s = w.layers[i];
    lp[i] = {s.wqkv, s.waproj, s.wfc, s.wmproj, s.bqkv, s.baproj, s.bfc, s.bmproj, s.ln1w, s.ln1b, s.ln2w, s.ln2b};
  }
  if (hipMalloc(&pl->layers_dev, sizeof(LayerPtrs) * L) != hipSuccess) return pl;
  if (hipMemcpy(pl->layers_dev, lp.data(), sizeof(LayerPtrs) * L, hipMemcpyHostToDevice) != hipSuccess) return pl;
  p.layers = pl->layers_dev;
  p.wte = w.wte;
  p.wpe = w.wpe;
  p.lnfw = w.lnfw;
  p.lnfb = w.lnfb;
  p.L = L;
  p.d = d;
  p.H = H;
  p.V = V;
  p.P = (int)w.cfg.n_positions;
  p.eps = w.cfg.layer_norm_epsilon;
  p.wtype = w.wtype;
  {
    // per-helper attention positions: ceil(ceil(P / C) / NA) <= ATT_POS_MAX for the smallest C
    const int capc = std::max(1, std::min(CMAX, std::min(MAX_ITEMS / H, G / H)));
    const int per = ((p.P + capc - 1) / capc + NA - 1) / NA;
    if (per > ATT_POS_MAX) return pl;
  }
  pl->G = G;
  pl->maxseg = maxseg;
  return pl;
}

void persistent_plan_destroy(PersistentPlan* pl) {
  if (!pl) return;
  if (pl->layers_dev) hipFree(pl->layers_dev);
  delete pl;
}

bool persistent_supported(const PersistentPlan* pl, int batch) {
  if (!pl || pl->maxseg == 0 || batch != 1) return false;
  const char* off = getenv("RTG_DISABLE_PERSISTENT");
  return !(off && off[0] == '1');
}

PersistentState* persistent_state_create(PersistentPlan* pl, float* kcache, float* vcache, int batch,
                                         uint32_t* token_dev, int* pos_dev, float* logits,
                                         unsigned long long* keys) {
  if (!persistent_supported(pl, batch)) return nullptr;
  PersistentState* s = new PersistentState();
  s->plan = pl;
  s->p = pl->base;
  Params& p = s->p;
  const int d = p.d, H = p.H;
  p.o_qkv = 0;
  p.o_att = 3 * d;
  p.o_x2 = p.o_att + MAX_ITEMS * ITEM_WORDS;
  p.o_h = p.o_x2 + d;
  p.o_x3 = p.o_h + 4 * d;
  p.lw = (p.o_x3 + d + 63) / 64 * 64;
  (void)H;
  const size_t words = (size_t)p.lw * p.L;
  if (hipMalloc(&s->tags, words * 8) != hipSuccess || hipMalloc(&s->epoch, 256) != hipSuccess ||
      hipMalloc(&s->err, 256) != hipSuccess) {
    persistent_state_destroy(s);
    return nullptr;
  }
  hipMemset(s->tags, 0, words * 8);
  const unsigned one = 1;
  hipMemcpy(s->epoch, &one, 4, hipMemcpyHostToDevice);
  hipMemset(s->err, 0, 256);
  p.tag = s->tags;
  p.epoch = s->epoch;
  p.err = s->err;
  p.kc = kcache;
  p.vc = vcache;
  p.kv_layer = (long)H * p.P * HD;
  p.token = token_dev;
  p.pos = pos_dev;
  p.logits = logits;
  p.keys = keys;
  return s;
}

void persistent_state_destroy(PersistentState* s) {
  if (!s) return;
  if (s->tags) hipFree(s->tags);
  if (s->epoch) hipFree(s->epoch);
  if (s->err) hipFree(s->err);
  delete s;
}

unsigned* persistent_epoch(PersistentState* s) { return s ? s->epoch : nullptr; }
unsigned* persistent_err(PersistentState* s) { return s ? s->err : nullptr; }

hipError_t persistent_decode_step(PersistentState* s, hipStream_t stream, bool cooperative) {
  void* args[] = {&s->p};
  const PersistentPlan* pl = s->plan;
  const bool bf = pl->w.wtype == W_BF16;
  void* fn;
  if (pl->maxseg == 8) fn = bf ? (void*)decode_step_kernel<W_BF16, 8> : (void*)decode_step_kernel<W_F32, 8>;
  else fn = bf ? (void*)decode_step_kernel<W_BF16, 16> : (void*)decode_step_kernel<W_F32, 16>;
  if (cooperative) return hipLaunchCooperativeKernel(fn, dim3(pl->G), dim3(NTHREADS), args, 0, stream);
  // Graph-captured path: a plain launch of exactly one workgroup per CU (the
  // kernel's LDS footprint admits no second one), all co-resident on an
  // otherwise idle device; every wait is bounded should that not hold.
  return hipLaunchKernel(fn, dim3(pl->G), dim3(NTHREADS), args, 0, stream);
}

}  // namespace rtg
