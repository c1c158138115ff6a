// Device side of the tiled persistent decode step (batch 1, f32 weights,
// n_head <= 16, contexts up to LMAX positions). One launch runs a whole
// forward_cached(&[token]) + argmax (rusttorch-core/src/nn/gpt2.rs:358-399,
// 477-538, 858-868) on all 256 CUs.
//
// Every layer matrix is cut into a 16 x 16 grid of weight tiles and
// workgroup w owns tile (R, C) = (w >> 4, w & 15) of each: the rows of row
// block R over the inputs of column block C. A workgroup's GEMV therefore
// needs only one column block of its input, and produces partial sums that
// the consumers of the next phase add up themselves. Each exchange is then a
// gather from 16 producers (12 for the attention projection) instead of an
// all-gather from all 256 workgroups:
//   E1  x   block C   <- mlp c_proj partials of tiles (C, 0..15)    48 rows
//   E2  q,k,v head R  <- c_attn partials of tiles (R, 0..15)       192 rows
//   E4  x2  block C   <- attn c_proj partials of tiles (0..H-1, C)  48 rows
//   E5  h   block C   <- c_fc partials of tiles (C, 0..15)         192 rows
// The attention of head R runs in every workgroup of grid row R (each
// needs the whole head output for its projection tile), so the attention
// output itself is never exchanged: four exchanges per layer.
//
// LayerNorm is folded into the GEMV that follows it, centred on exact block
// statistics: the producer of tile (R, C) multiplies (x - mu_C) * g over
// its column block, where mu_C is the block's own mean, and publishes mu_C
// and M2_C = sum (x - mu_C)^2 with its partials. A consumer merges the 16
// blocks' statistics (Chan et al.'s pairwise update, the two-pass mean and
// variance of gpt2.rs:636-666 in exact arithmetic) and finishes
//   LN(x) W + b = inv_std (sum_C P_C + sum_C (mu_C - mean) s_C) + c
// with s_C = sum_{k in C} W[k] g[k] and c = bias + sum_k W[k] b[k]
// precomputed in double. No term cancels a large mean: the partials are
// taken about their block mean and the correction only carries the spread
// of the block means.
//
// The exchange protocol is the one of decode_persistent_kernel.h: 64-bit
// tagged words {epoch, f32} written once per step into per-(layer, phase)
// regions with one slot of whole 128-byte lines per producer, polled with
// agent-scope loads; every wait is bounded and sets *err on timeout.
//
// Waves: 0 leader (E1, E4, block statistics, finalize), 1-2 helpers (E2,
// E5 and the attention with the leader), 3-7 GEMV waves (one task per lane:
// a row, or a quarter of a row reduced over four lanes; weights in registers
// one phase ahead; every lane stores its own result).
#pragma once
#include "decode_persistent_kernel.h"

namespace rtg {
namespace tk {

using pk::f4v;
using pk::u64;

constexpr int G = 256;   // workgroups = CUs of an MI355X
constexpr int GS = 16;   // grid side
constexpr int NGLUE = 3;
constexpr int NGEMV = 5;
constexpr int NTHREADS = (NGLUE + NGEMV) * 64;
constexpr int HD = 64;
constexpr int LMAX = pk::KVS;  // longest context (cached positions + the new one): one LDS window per attention wave
constexpr int RB = 4;          // LM-head rows per register batch of a GEMV wave
#ifndef TK_PACE
#define TK_PACE 2
#endif
#ifndef TK_SLEEP
#define TK_SLEEP 2
#endif

enum { PQ = 0, PP = 1, PF = 2, PM = 3, PL = 4 };

__host__ __device__ constexpr int lines(int words) { return (words + 15) / 16 * 16; }

template <int D_, int V_>
struct TCfg {
  static constexpr int D = D_, V = V_, H = D_ / HD;
  static constexpr int CB = D / GS;       // column block of the residual stream
  static constexpr int HB = 4 * D / GS;   // column block of the MLP hidden vector = c_fc row block
  static constexpr int QR = 3 * HD;       // q, k, v rows of one head (head-major row order)
  static constexpr int NV = CB / 4;       // float4 of a c_attn / c_fc / mlp c_proj task
  static constexpr int NVP = HD / 16;     // float4 of an attn c_proj task (16 of the head's 64 columns)
  static constexpr int NT_Q = QR, NT_P = 4 * CB, NT_F = HB, NT_M = 4 * CB;
  static constexpr int NT_MAX = NT_Q > NT_F ? (NT_Q > NT_M ? NT_Q : NT_M) : (NT_F > NT_M ? NT_F : NT_M);
  static constexpr int NTW = (NT_MAX + 63) / 64;  // GEMV waves with layer tasks
  static constexpr int NVL = D / 256;             // float4 per lane of one LM-head row
  static constexpr int NB = NV > RB * NVL ? NV : RB * NVL;
  // slots: partials, then (for c_attn and c_fc) the producer's block mean and M2
  static constexpr int SQ = lines(QR + 2), SP = lines(CB), SF = lines(HB + 2), SM = lines(CB), SX = lines(CB + 2);
  static constexpr int LMR = (V + G - 1) / G;  // LM-head rows per workgroup
  static constexpr int NXV = (D + 64 * NGLUE - 1) / (64 * NGLUE);  // residual values per glue lane (LM input)
  static_assert(D % 256 == 0 && H <= GS, "width");
  static_assert(CB % 4 == 0 && CB <= 64, "column block: one leader lane per row");
  static_assert(QR == 64 * NGLUE, "one glue lane per q/k/v row");
  static_assert(NT_P <= 64 * NGEMV && NT_MAX <= 64 * NGEMV, "one task per GEMV lane");
  static_assert(NVP <= NB, "register buffer");
};

struct TLayer {
  const f4v *wq, *wp, *wf, *wm;    // weight tiles (layout in decode_tile.hip)
  const float *sq, *cq, *sf, *cf;  // folded LayerNorm: s [rows][16] and c [rows]; c_attn rows head-major
  const float *bp, *bm, *g1, *g2;  // attn c_proj bias, mlp c_proj bias, LN1 and LN2 gains
};

struct TParams {
  const TLayer* layers;
  const float* wte;  // [V][D]: embedding and tied LM head
  const float* wpe;
  const float* gf;   // ln_f gain
  const float* cl;   // cl[v] = sum_k wte[v][k] ln_f.bias[k]
  int L, P;
  float eps;
  float* kc;  // [L][H][P][HD]
  float* vc;
  long kv_layer;
  uint32_t* token;
  int* pos;
  uint32_t* ids_out;
  int* step;
  unsigned* done;
  unsigned* epoch;
  u64* tag;  // tagged words: lw per layer, then the LM-head input slots at o_x
  long lw;
  long o_q, o_p, o_f, o_m, o_x;
  float* logits;
  u64* keys;
  unsigned* err;
  u64* trace;
  const void* dummy;  // >= 1 KiB of zeros
};

template <int D>
struct TSmem {
  float u[D / GS];    // c_attn input (x - mu) * g1 of the column block
  float u2[D / GS];   // c_fc input
  float xb[D / GS];   // residual x of the block (layer input)
  float x2b[D / GS];  // residual after attention
  float qkv[3 * HD];  // q, k_new, v_new of the head
  float a[HD];        // attention output of the head (attn c_proj input)
  float hb[4 * D / GS];  // gelu output of the hidden block (mlp c_proj input)
  float uf[D];           // LM-head input (x - mean) * g_f
  float kv_k[pk::KVS * HD], kv_v[pk::KVS * HD];
  float att_part[NGLUE][HD + 2];
  float lm_inv;
  u64 wkey[NGEMV];
  // in_ready[phase]: inputs delivered (PQ, PP, PF: one count per layer;
  // PM, PL: one per glue wave); glue_cnt: glue barrier; att_cnt: attention
  // waves finished; gemv_done: LM-head waves finished
  unsigned in_ready[5], glue_cnt, att_cnt, gemv_done;
  u64 trace_t0;
  unsigned trace_rel[pk::TRACE_N];
  // keeps the footprint above half the CU's LDS: one workgroup per CU
  float pad[4096];
};

#define TK_TRACE(p, idx, lane)                                               \
  do {                                                                       \
    if ((p).trace && (lane) == 0 && (idx) >= 0 && (idx) < pk::TRACE_N)       \
      sm.trace_rel[(idx)] = (unsigned)(wall_clock64() - sm.trace_t0) | 1u;   \
  } while (0)

// Mean and M2 of the CB values x held by lanes 0..CB-1 (two-pass within
// the block); d = x - mean in those lanes, 0 elsewhere.
template <int CB>
__device__ __forceinline__ void block_stats(float x, int lane, float& mu, float& m2, float& d) {
  mu = pk::wave_sum_all(lane < CB ? x : 0.f) / (float)CB;
  d = lane < CB ? x - mu : 0.f;
  m2 = pk::wave_sum_all(d * d);
}

// Global mean and 1 / sqrt(var + eps) of a D-vector from its GS blocks'
// statistics: lane c < GS holds mu_c, lane GS + c holds M2_c. Chan's merge
// of equal-size blocks: M2 = sum M2_c + CB sum (mu_c - mean)^2.
template <int D>
__device__ __forceinline__ void merge_stats(float v, int lane, float eps, float& mean, float& inv_std) {
  constexpr int CB = D / GS;
  mean = pk::wave_sum_all(lane < GS ? v : 0.f) / (float)GS;
  const float dm = lane < GS ? v - mean : 0.f;
  const float m2 = lane >= GS && lane < 2 * GS ? v : 0.f;
  const float tot = pk::wave_sum_all(m2 + (float)CB * dm * dm);
  inv_std = 1.0f / sqrtf(tot / (float)D + eps);
}

// sum_c (mu_c - mean) s[c] with mu_c in lane c of `stat` (wave-uniform
// broadcast) and s the row's 16 per-block gain sums.
__device__ __forceinline__ float block_correction(float stat, float mean, const float* s) {
  float corr = 0.f;
#pragma unroll
  for (int c = 0; c < GS; ++c) {
    const float mu = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(stat), c));
    corr += (mu - mean) * s[c];
  }
  return corr;
}

__device__ __forceinline__ void glue_barrier_t(unsigned* cnt, unsigned& gen, int lane, unsigned* err) {
  ++gen;
  pk::lds_release();
  if (lane == 0) pk::lds_add(cnt, 1);
  pk::lds_wait_ge(cnt, gen * NGLUE, err);
}

// ---------------------------------------------------------------------------
// Glue waves (leader gw = 0, helpers 1..2)
// ---------------------------------------------------------------------------
template <class C>
__device__ __forceinline__ void tglue(const TParams& p, TSmem<C::D>& sm, int gw, int lane0, int len, unsigned tag,
                                      uint32_t tok) {
  constexpr int D = C::D, CB = C::CB, HB = C::HB, QR = C::QR;
  const int w = blockIdx.x, R = w >> 4, Cc = w & 15;
  const bool attn = R < C::H;
  const bool leader = gw == 0;
  int lane = lane0;
  int g = gw * 64 + lane;
  const int pos = len - 1;
  unsigned gen = 0;
  // attention rows of this wave: cached positions [h0, h1) of head R
  const int per = (pos + NGLUE - 1) / NGLUE;
  const int h0 = min(pos, gw * per), h1 = min(pos, h0 + per);
  float* ldsK = sm.kv_k + gw * pk::KVW * HD;
  float* ldsV = sm.kv_v + gw * pk::KVW * HD;
  const long kv_head = (long)R * p.P * HD;
  if (attn && h1 > h0) pk::stage_rows(p.kc + kv_head, p.vc + kv_head, h0, h1 - h0, ldsK, ldsV, lane);
  const __attribute__((address_space(4))) TLayer* LPs = PK_C(TLayer, p.layers);
  for (int l = 0; l <= p.L; ++l) {
    // Per-iteration copies of the lane index: they keep the compiler from
    // hoisting every phase's polling addresses out of the layer loop, where
    // they would hold ~130 registers across the whole step (and spill).
    lane = lane0;
    asm volatile("" : "+v"(lane));
    g = gw * 64 + lane;
    // ---- E1 (leader): the layer input's column block Cc ----
    float x = 0.f, mu = 0.f, m2 = 0.f, dx = 0.f;
    if (leader) {
      if (l == 0) {
        if (lane < CB)
          x = PK_G(float, p.wte)[(long)tok * D + CB * Cc + lane] + PK_G(float, p.wpe)[(long)pos * D + CB * Cc + lane];
      } else {
        const u64* src = p.tag + (long)(l - 1) * p.lw + p.o_m;
        int idx[GS];
#pragma unroll
        for (int c = 0; c < GS; ++c) idx[c] = (GS * Cc + c) * C::SM + lane;
        float v[GS];
        pk::poll_words<GS>(src, idx, lane < CB ? GS : 0, tag, v, p.err);
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < GS; ++c) s += v[c];
        // x3 = x2 + (mlp + bias), gpt2.rs:534-537
        if (lane < CB) x = sm.x2b[lane] + (s + PK_G(float, LPs[l - 1].bm)[CB * Cc + lane]);
      }
      block_stats<CB>(x, lane, mu, m2, dx);
      TK_TRACE(p, 8 * l, lane);
    }
    if (l == p.L) {
      // ---- LM-head input: every workgroup needs the whole x3; the
      //      workgroups of grid row 0 publish their blocks ----
      if (leader && R == 0) {
        u64* dst = p.tag + p.o_x + (long)Cc * C::SX;
        if (lane < CB) pk::tstore(dst + lane, x, tag);
        if (lane < 2) pk::tstore(dst + CB + lane, lane == 0 ? mu : m2, tag);
      }
      // lane g holds values g + 192 k (indices past D repeat the last one),
      // lanes < 32 also poll the 16 blocks' statistics
      int idx[C::NXV + 1];
#pragma unroll
      for (int k = 0; k < C::NXV; ++k) {
        const int v = min(g + 64 * NGLUE * k, D - 1);
        idx[k] = (v / CB) * C::SX + v % CB;
      }
      idx[C::NXV] = (lane & 15) * C::SX + CB + (lane >> 4);
      float v[C::NXV + 1];
      pk::poll_words<C::NXV + 1>(p.tag + p.o_x, idx, lane < 2 * GS ? C::NXV + 1 : C::NXV, tag, v, p.err);
      const float stat = lane < 2 * GS ? v[C::NXV] : 0.f;
      float mean, inv;
      merge_stats<D>(stat, lane, p.eps, mean, inv);
#pragma unroll
      for (int k = 0; k < C::NXV; ++k) {
        const int vi = g + 64 * NGLUE * k;
        if (vi < D) sm.uf[vi] = (v[k] - mean) * PK_G(float, p.gf)[vi];
      }
      if (leader && lane == 0) sm.lm_inv = inv;
      pk::lds_release();
      if (lane == 0) pk::lds_add(&sm.in_ready[PL], 1);
      if (leader) TK_TRACE(p, 8 * p.L + 1, lane);
      break;
    }
    const __attribute__((address_space(4))) TLayer& LP = LPs[l];
    u64* T = p.tag + (long)l * p.lw;
    if (leader) {
      if (lane < CB) {
        sm.xb[lane] = x;
        sm.u[lane] = dx * PK_G(float, LP.g1)[CB * Cc + lane];
      }
      if (attn && lane < 2) pk::tstore(T + p.o_q + (long)w * C::SQ + QR + lane, lane == 0 ? mu : m2, tag);
      pk::lds_release();
      if (lane == 0) pk::lds_add(&sm.in_ready[PQ], 1);
    }
    // ---- E2 + attention (grid rows < H): head R ----
    if (attn) {
      const float* srow = LP.sq + (long)(QR * R + g) * GS;
      float s[GS];
#pragma unroll
      for (int c = 0; c < GS; c += 4) {
        const f4v t4 = PK_G(f4v, srow + c)[0];
        s[c] = t4.x; s[c + 1] = t4.y; s[c + 2] = t4.z; s[c + 3] = t4.w;
      }
      const float cq = PK_G(float, LP.cq)[QR * R + g];
      int idx[GS + 1];
#pragma unroll
      for (int c = 0; c < GS; ++c) idx[c] = (GS * R + c) * C::SQ + g;
      idx[GS] = (GS * R + (lane & 15)) * C::SQ + QR + (lane >> 4);
      float v[GS + 1];
      pk::poll_words<GS + 1>(T + p.o_q, idx, lane < 2 * GS ? GS + 1 : GS, tag, v, p.err);
      const float stat = lane < 2 * GS ? v[GS] : 0.f;
      float mean, inv;
      merge_stats<D>(stat, lane, p.eps, mean, inv);
      float z = 0.f;
#pragma unroll
      for (int c = 0; c < GS; ++c) z += v[c];
      const float val = inv * (z + block_correction(stat, mean, s)) + cq;
      sm.qkv[g] = val;
      if (Cc == 0 && g >= HD) {  // k, v of the new token into the cache (LayerKVCache::append, gpt2.rs:500-514)
        float* base = (g < 2 * HD ? p.kc : p.vc) + (long)l * p.kv_layer + ((long)R * p.P + pos) * HD;
        PK_GW(float, base)[g < 2 * HD ? g - HD : g - 2 * HD] = val;
      }
      if (leader) TK_TRACE(p, 8 * l + 1, lane);
      glue_barrier_t(&sm.glue_cnt, gen, lane, p.err);
      // multi_head_attention_cached, gpt2.rs:772-834: rows [h0, h1) of this
      // wave from its LDS window, the new row on the last wave
      const int grp = lane >> 4, dq = (lane & 15) * 4;
      const float4 q4 = *reinterpret_cast<const float4*>(sm.qkv + dq);
      float m = -INFINITY, lsum = 0.f;
      float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (h1 > h0) {
        pk::wait_vm_all();
        pk::att_window(ldsK, ldsV, h1 - h0, q4, grp, dq, m, lsum, o4);
      }
      if (gw == NGLUE - 1) {
        const float4 k = *reinterpret_cast<const float4*>(sm.qkv + HD + dq);
        const float4 vv = *reinterpret_cast<const float4*>(sm.qkv + 2 * HD + dq);
        const float sc = pk::row16_sum(q4.x * k.x + q4.y * k.y + q4.z * k.z + q4.w * k.w) * 0.125f;
        const float mn = fmaxf(m, sc);
        const float corr = m == -INFINITY ? 0.f : pk::fexp(m - mn);
        const float pj = grp == 0 ? pk::fexp(sc - mn) : 0.f;
        lsum = lsum * corr + pj;
        o4.x = o4.x * corr + pj * vv.x;
        o4.y = o4.y * corr + pj * vv.y;
        o4.z = o4.z * corr + pj * vv.z;
        o4.w = o4.w * corr + pj * vv.w;
        m = mn;
      }
      lsum = pk::xor32_sum(pk::xor16_sum(lsum));
      o4.x = pk::xor32_sum(pk::xor16_sum(o4.x));
      o4.y = pk::xor32_sum(pk::xor16_sum(o4.y));
      o4.z = pk::xor32_sum(pk::xor16_sum(o4.z));
      o4.w = pk::xor32_sum(pk::xor16_sum(o4.w));
      if (lane < 16) {
        sm.att_part[gw][2 + dq + 0] = o4.x;
        sm.att_part[gw][2 + dq + 1] = o4.y;
        sm.att_part[gw][2 + dq + 2] = o4.z;
        sm.att_part[gw][2 + dq + 3] = o4.w;
      }
      if (lane == 0) {
        sm.att_part[gw][0] = m;
        sm.att_part[gw][1] = lsum;
      }
      pk::lds_release();
      unsigned arrived = 0;
      if (lane == 0) arrived = __hip_atomic_fetch_add(&sm.att_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      arrived = __builtin_amdgcn_readlane(arrived, 0);
      if (arrived == (unsigned)((l + 1) * NGLUE - 1)) {
        // the last wave merges the three partial softmaxes: the head output
        pk::lds_acquire();
        float M = -INFINITY;
#pragma unroll
        for (int q = 0; q < NGLUE; ++q) M = fmaxf(M, sm.att_part[q][0]);
        float Ls = 0.f, o = 0.f;
#pragma unroll
        for (int q = 0; q < NGLUE; ++q) {
          const float mw = sm.att_part[q][0];
          if (mw == -INFINITY) continue;
          const float f = pk::fexp(mw - M);
          Ls += sm.att_part[q][1] * f;
          o += sm.att_part[q][2 + lane] * f;
        }
        sm.a[lane] = o / Ls;
        pk::lds_release();
        if (lane == 0) pk::lds_add(&sm.in_ready[PP], 1);
        TK_TRACE(p, 8 * l + 2, lane);
      }
      if (l + 1 < p.L && h1 > h0) {  // the window is free again: the next layer's rows
        const long nl = (long)(l + 1) * p.kv_layer + kv_head;
        pk::stage_rows(p.kc + nl, p.vc + nl, h0, h1 - h0, ldsK, ldsV, lane);
      }
    }
    // ---- E4 (leader): x2 block Cc = x + (attn c_proj + bias) ----
    if (leader) {
      int idx[GS];
#pragma unroll
      for (int h = 0; h < GS; ++h) idx[h] = h < C::H ? (GS * h + Cc) * C::SP + lane : 0;
      float v[GS];
      pk::poll_words<GS>(T + p.o_p, idx, lane < CB ? C::H : 0, tag, v, p.err);
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < C::H; ++h) s += v[h];
      const float x2 = lane < CB ? sm.xb[lane] + (s + PK_G(float, LP.bp)[CB * Cc + lane]) : 0.f;
      float mu2, m22, d2;
      block_stats<CB>(x2, lane, mu2, m22, d2);
      if (lane < CB) {
        sm.x2b[lane] = x2;
        sm.u2[lane] = d2 * PK_G(float, LP.g2)[CB * Cc + lane];
      }
      if (lane < 2) pk::tstore(T + p.o_f + (long)w * C::SF + HB + lane, lane == 0 ? mu2 : m22, tag);
      pk::lds_release();
      if (lane == 0) pk::lds_add(&sm.in_ready[PF], 1);
      TK_TRACE(p, 8 * l + 3, lane);
    }
    // ---- E5 (glue waves): h block Cc = gelu_new(LN2(x2) c_fc + bias) ----
    for (int j = g; j < HB; j += 64 * NGLUE) {
      const float* srow = LP.sf + (long)(HB * Cc + j) * GS;
      float s[GS];
#pragma unroll
      for (int c = 0; c < GS; c += 4) {
        const f4v t4 = PK_G(f4v, srow + c)[0];
        s[c] = t4.x; s[c + 1] = t4.y; s[c + 2] = t4.z; s[c + 3] = t4.w;
      }
      const float cf = PK_G(float, LP.cf)[HB * Cc + j];
      int idx[GS + 1];
#pragma unroll
      for (int c = 0; c < GS; ++c) idx[c] = (GS * Cc + c) * C::SF + j;
      idx[GS] = (GS * Cc + (lane & 15)) * C::SF + HB + (lane >> 4);
      float v[GS + 1];
      pk::poll_words<GS + 1>(T + p.o_f, idx, lane < 2 * GS ? GS + 1 : GS, tag, v, p.err);
      const float stat = lane < 2 * GS ? v[GS] : 0.f;
      float mean, inv;
      merge_stats<D>(stat, lane, p.eps, mean, inv);
      float z = 0.f;
#pragma unroll
      for (int c = 0; c < GS; ++c) z += v[c];
      sm.hb[j] = pk::gelu_new(inv * (z + block_correction(stat, mean, s)) + cf);
    }
    pk::lds_release();
    if (lane == 0) pk::lds_add(&sm.in_ready[PM], 1);
    if (leader) TK_TRACE(p, 8 * l + 4, lane);
  }
  // ---- argmax and the end of the step (gpt2.rs:431-437, 858-868) ----
  if (leader) {
    pk::lds_wait_ge(&sm.gemv_done, NGEMV, p.err);
    u64 best = 0ull;
#pragma unroll
    for (int q = 0; q < NGEMV; ++q) best = sm.wkey[q] > best ? sm.wkey[q] : best;
    TK_TRACE(p, 8 * p.L + 2, lane);
    u64 prev = 0ull;
    if (lane == 0 && best != 0ull)
      prev = __hip_atomic_fetch_max(PK_GW(u64, p.keys), best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The last workgroup to arrive finishes the step: each workgroup's key
    // update has completed (the returned value) before it counts itself.
    if (lane == 0) {
      asm volatile("" : : "v"(prev));
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
      const unsigned arrived =
          __hip_atomic_fetch_add(PK_GW(unsigned, p.done), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// ---------------------------------------------------------------------------
// GEMV waves
// ---------------------------------------------------------------------------

// Dot product of a task's NX float4 with 4 * NX consecutive LDS floats x.
template <int NX, int NB>
__device__ __forceinline__ float task_dot(const f4v (&buf)[NB], const float* x) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const float4 xv = *reinterpret_cast<const float4*>(x + 4 * i);
    a += buf[i].x * xv.x + buf[i].y * xv.y + buf[i].z * xv.z + buf[i].w * xv.w;
  }
  return a;
}

// Sum over the four lanes of a quad (DPP quad_perm [1,0,3,2], then [2,3,0,1]).
__device__ __forceinline__ float quad_sum(float v) {
  v += pk::dpp_mov<0xB1>(v);
  v += pk::dpp_mov<0x4E>(v);
  return v;
}

template <class C>
__device__ __forceinline__ void tgemv(const TParams& p, TSmem<C::D>& sm, int tw, int lane, unsigned tag) {
  constexpr int D = C::D, V = C::V, NB = C::NB, NV = C::NV, NVP = C::NVP, NVL = C::NVL, CB = C::CB;
  const int w = blockIdx.x, R = w >> 4;
  const bool attn = R < C::H;
  const int t = tw * 64 + lane;
  const f4v* dz = reinterpret_cast<const f4v*>(p.dummy) + lane;
  const __attribute__((address_space(4))) TLayer* LPs = PK_C(TLayer, p.layers);
  f4v A[NB], B[NB];
  // Loads are always issued (a lane without a task, or a tile this
  // workgroup does not own, reads the zero page), so every path through the
  // layer loop issues the same load sequence and each compute waits only
  // for its own buffer.
  // Refills are paced: a sleep between loads while the wave's next compute
  // is not due (*ready < next), so that the weight loads in flight do not
  // queue ahead of the glue waves' polls in this CU's memory path; once the
  // next input is there the remaining loads go out back to back. Only the
  // sleeps depend on timing, the loads keep their order.
  auto load_tile = [&](f4v(&buf)[NB], const f4v* tile, int NT, int nv, bool own, unsigned* ready, unsigned next) {
    bool go = false;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const f4v* ptr = own && i < nv && t < NT ? tile + (long)i * NT + t : dz;
      buf[i] = __builtin_nontemporal_load(PK_G(f4v, ptr));
      if (TK_PACE > 0 && i + 1 < NB && !go)
        for (int q = 0; q < TK_PACE; ++q) {
          if (pk::lds_load(ready) >= next) {
            go = true;
            break;
          }
          __builtin_amdgcn_s_sleep(TK_SLEEP);
        }
    }
  };
  // LM head (tied wte, gpt2.rs:392-396): rows v0 + tw + NGEMV * k of this
  // workgroup, RB rows per batch
  const int v0 = w * C::LMR;
  const int nrows = max(0, min(C::LMR, V - v0));
  const int nk = nrows > tw ? (nrows - tw + NGEMV - 1) / NGEMV : 0;
  const int nbat = (nk + RB - 1) / RB;
  const f4v* wte4 = reinterpret_cast<const f4v*>(p.wte);
  auto load_lm = [&](f4v(&buf)[NB], int b) {
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int m = 0; m < NVL; ++m) {
        const int k = RB * b + r;
        const f4v* ptr = k < nk ? wte4 + (long)(v0 + tw + NGEMV * k) * (D / 4) + m * 64 + lane : dz;
        buf[r * NVL + m] = PK_G(f4v, ptr)[0];
      }
  };
  if (tw < C::NTW) {
    const long wq = (long)w * NV * C::NT_Q, wp = (long)w * NVP * C::NT_P;
    const long wf = (long)w * NV * C::NT_F, wm = (long)w * NV * C::NT_M;
    load_tile(A, LPs[0].wq + wq, C::NT_Q, NV, attn, &sm.in_ready[PQ], 0u);
    load_tile(B, LPs[0].wp + wp, C::NT_P, NVP, attn, &sm.in_ready[PQ], 0u);
    for (int l = 0; l < p.L; ++l) {
      u64* T = p.tag + (long)l * p.lw;
      const unsigned n1 = (unsigned)(l + 1);
      if (attn) {  // c_attn tile: q/k/v rows of head R over column block C
        pk::lds_wait_ge(&sm.in_ready[PQ], n1, p.err);
        if (tw == 0) TK_TRACE(p, 800 + 8 * l, lane);
        const float r = task_dot<NV>(A, sm.u);
        if (t < C::NT_Q) pk::tstore(T + p.o_q + (long)w * C::SQ + t, r, tag);
        if (tw == 0) TK_TRACE(p, 801 + 8 * l, lane);
      }
      // paced until the next compute's input: attn c_proj, or c_fc itself
      load_tile(A, LPs[l].wf + wf, C::NT_F, NV, true, &sm.in_ready[attn ? PP : PF], n1);
      if (attn) {  // attn c_proj tile: rows of block C over head R's columns
        pk::lds_wait_ge(&sm.in_ready[PP], n1, p.err);
        if (tw == 0) TK_TRACE(p, 802 + 8 * l, lane);
        const int q = t & 3;
        const float r = quad_sum(task_dot<NVP>(B, sm.a + 16 * q));
        if (t < C::NT_P && q == 0) pk::tstore(T + p.o_p + (long)w * C::SP + (t >> 2), r, tag);
        if (tw == 0) TK_TRACE(p, 803 + 8 * l, lane);
      }
      load_tile(B, LPs[l].wm + wm, C::NT_M, NV, true, &sm.in_ready[PF], n1);  // next: c_fc
      {  // c_fc tile
        pk::lds_wait_ge(&sm.in_ready[PF], n1, p.err);
        if (tw == 0) TK_TRACE(p, 804 + 8 * l, lane);
        const float r = task_dot<NV>(A, sm.u2);
        if (t < C::NT_F) pk::tstore(T + p.o_f + (long)w * C::SF + t, r, tag);
        if (tw == 0) TK_TRACE(p, 805 + 8 * l, lane);
      }
      if (l + 1 < p.L) load_tile(A, LPs[l + 1].wq + wq, C::NT_Q, NV, attn, &sm.in_ready[PM], NGLUE * n1);
      else load_lm(A, 0);
      {  // mlp c_proj tile: quarter (t & 3) of row t >> 2's hidden columns
        pk::lds_wait_ge(&sm.in_ready[PM], NGLUE * n1, p.err);
        if (tw == 0) TK_TRACE(p, 806 + 8 * l, lane);
        const int q = t & 3;
        const float r = quad_sum(task_dot<NV>(B, sm.hb + CB * q));
        if (t < C::NT_M && q == 0) pk::tstore(T + p.o_m + (long)w * C::SM + (t >> 2), r, tag);
        if (tw == 0) TK_TRACE(p, 807 + 8 * l, lane);
      }
      if (l + 1 < p.L)
        load_tile(B, LPs[l + 1].wp + wp, C::NT_P, NVP, attn, &sm.in_ready[attn ? PQ : PF], n1 + 1);
      else load_lm(B, 1);
    }
  } else {
    load_lm(A, 0);
    load_lm(B, 1);
  }
  pk::lds_wait_ge(&sm.in_ready[PL], NGLUE, p.err);
  const float inv = sm.lm_inv;
  float4 xv[NVL];
#pragma unroll
  for (int m = 0; m < NVL; ++m) xv[m] = *reinterpret_cast<const float4*>(sm.uf + 4 * (m * 64 + lane));
  u64 best = 0ull;
  auto lm_batch = [&](const f4v(&buf)[NB], int b) {
    float s[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float a = 0.f;
#pragma unroll
      for (int m = 0; m < NVL; ++m) {
        const f4v wv = buf[r * NVL + m];
        a += wv.x * xv[m].x + wv.y * xv[m].y + wv.z * xv[m].z + wv.w * xv[m].w;
      }
      s[r] = a;
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) s[r] = pk::wave_sum_all(s[r]);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int k = RB * b + r;
      if (k < nk) {
        const int v = v0 + tw + NGEMV * k;
        const float logit = inv * s[r] + PK_G(float, p.cl)[v];
        if (lane == r) PK_GW(float, p.logits)[v] = logit;
        const u64 key = argmax_key(logit, (uint32_t)v);  // -inf and NaN give 0: they never win
        best = key > best ? key : best;
      }
    }
  };
  for (int b = 0; b < nbat; b += 2) {
    lm_batch(A, b);
    load_lm(A, b + 2);
    lm_batch(B, b + 1);
    load_lm(B, b + 3);
  }
  if (lane == 0) sm.wkey[tw] = best;
  pk::lds_release();
  if (lane == 0) pk::lds_add(&sm.gemv_done, 1);
}

template <int D, int V>
__global__ __launch_bounds__(NTHREADS) void decode_tile_kernel(TParams p) {
  typedef TCfg<D, V> C;
  __shared__ TSmem<D> sm;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (threadIdx.x == 0) {
    for (int i = 0; i < 5; ++i) sm.in_ready[i] = 0;
    sm.glue_cnt = 0;
    sm.att_cnt = 0;
    sm.gemv_done = 0;
    sm.trace_t0 = wall_clock64();
  }
  if (p.trace)
    for (int i = threadIdx.x; i < pk::TRACE_N; i += NTHREADS) sm.trace_rel[i] = 0;
  __syncthreads();
  const int len = *PK_G(int, p.pos) + 1;
  const unsigned tag = *PK_G(unsigned, p.epoch);
  const uint32_t tok = *PK_G(uint32_t, p.token);
  if (wave < NGLUE) tglue<C>(p, sm, wave, lane, len, tag, tok);
  else tgemv<C>(p, sm, wave - NGLUE, lane, tag);
  if (p.trace) {
    __syncthreads();
    for (int i = threadIdx.x; i < pk::TRACE_N; i += NTHREADS) {
      const unsigned r = sm.trace_rel[i];
      PK_GW(u64, p.trace)[(long)blockIdx.x * pk::TRACE_STRIDE + i] = r ? sm.trace_t0 + r : 0ull;
    }
  }
}

}  // namespace tk
}  // namespace rtg
