// gfx950 kernels for the GPT-2 token loop: embedding, LayerNorm, decode GEMV
// with fused epilogues, attention over the KV cache (decode and causal
// prefill), argmax, and an fp32 MFMA GEMM for prefill.
//
// Each kernel states the reference function it computes (file:line in
// rusttorch-core/src/nn/gpt2.rs). Arithmetic is fp32 throughout; weights may
// be stored as bf16 and widened with the reference's bf16_to_f32 (bits << 16,
// nn/safetensors.rs:389-391).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "argmax_key.h"
#include "attn_core.h"
#include "bf16_split.h"
#include "gelu.h"
#include "kernels.h"

namespace rtg {

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block reduction over blockDim.x threads (multiple of 64, <= 1024). red has
// >= 16 floats of LDS. Returns the total to every thread.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red) {
  v = MAX ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
  for (int w = 1; w < nw; ++w) t = MAX ? fmaxf(t, red[w]) : t + red[w];
  return t;
}

// Load E consecutive weights (16 bytes) widened to f32.
template <int WT>
struct WVec;
template <>
struct WVec<W_F32> {
  static constexpr int E = 4;
  __device__ __forceinline__ static void load(const void* base, size_t idx, float* out) {
    float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + idx);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
};
template <>
struct WVec<W_BF16> {
  static constexpr int E = 8;
  __device__ __forceinline__ static void load(const void* base, size_t idx, float* out) {
    uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + idx);
    out[0] = __uint_as_float(v.x << 16); out[1] = __uint_as_float(v.x & 0xffff0000u);
    out[2] = __uint_as_float(v.y << 16); out[3] = __uint_as_float(v.y & 0xffff0000u);
    out[4] = __uint_as_float(v.z << 16); out[5] = __uint_as_float(v.z & 0xffff0000u);
    out[6] = __uint_as_float(v.w << 16); out[7] = __uint_as_float(v.w & 0xffff0000u);
  }
};

__device__ __forceinline__ float load_w1(const void* base, size_t idx, int wtype) {
  if (wtype == W_F32) return reinterpret_cast<const float*>(base)[idx];
  return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
}

// ---------------------------------------------------------------------------
// embedding (gpt2.rs:377-384: embedding_lookup(wte) + embedding_lookup(wpe) + add)
// ---------------------------------------------------------------------------

__global__ void embed_kernel(const void* __restrict__ wte, int wtype, const float* __restrict__ wpe,
                             const uint32_t* __restrict__ ids, int T, int pos0, const int* __restrict__ pos_dev,
                             int d, float* __restrict__ x) {
  const int r = blockIdx.x;
  const int pos = pos_dev ? *pos_dev : pos0 + (r % T);
  const size_t tok = ids[r];
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    x[(size_t)r * d + j] = load_w1(wte, tok * d + j, wtype) + wpe[(size_t)pos * d + j];
}

void launch_embed(hipStream_t s, const void* wte, int wtype, const float* wpe, const uint32_t* ids, int rows, int T,
                  int pos0, const int* pos_dev, int d, float* x) {
  embed_kernel<<<rows, 256, 0, s>>>(wte, wtype, wpe, ids, T, pos0, pos_dev, d, x);
}

// ---------------------------------------------------------------------------
// LayerNorm (gpt2.rs:636-666): two-pass mean / variance, one block per row.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps, int d,
                                                        float* __restrict__ out) {
  __shared__ float red[16];
  const float* row = x + (size_t)blockIdx.x * d;
  float s = 0.f;
  for (int j = threadIdx.x; j < d; j += blockDim.x) s += row[j];
  const float mean = block_reduce<false>(s, red) / (float)d;
  float v = 0.f;
  for (int j = threadIdx.x; j < d; j += blockDim.x) {
    float t = row[j] - mean;
    v += t * t;
  }
  const float var = block_reduce<false>(v, red) / (float)d;
  const float inv_std = 1.0f / sqrtf(var + eps);
  for (int j = threadIdx.x; j < d; j += blockDim.x)
    out[(size_t)blockIdx.x * d + j] = (row[j] - mean) * inv_std * w[j] + b[j];
}

// The same two-pass LayerNorm with one wave per row (4 rows per workgroup)
// for d % 4 == 0, d <= 2048: the row stays in registers (lane l holds the
// 16-byte chunks l, l + 64, ...), sums are wave reductions (DPP row sums, then
// the lane-16 / lane-32 swaps), no LDS and no barriers. The block-per-row
// kernel above needed three passes and two workgroup reductions per row
// (142 us for c4's 32768 x 1280, 2.4 TB/s).
constexpr int LNW_MAXC = 8;  // 16-byte chunks per lane: d <= 64 * 4 * 8
// full-wave sum in every lane on DPP and permlane swaps (no LDS traffic)
__device__ __forceinline__ float wave_sum_dpp(float v) { return xor32_sum_k(xor16_sum_k(row16_sum_k(v))); }

template <int NU>
__global__ __launch_bounds__(256) void layernorm_wave_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ b, float eps, int rows, int d,
                                                             float* __restrict__ out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= rows) return;  // wave-uniform
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)row * d);
  const int nc = d >> 2;  // 16-byte chunks of the row, NU per lane at most
  const float4* w4 = reinterpret_cast<const float4*>(w);
  const float4* b4 = reinterpret_cast<const float4*>(b);
  // the row, the gain and the bias in flight together (branch-free: chunks
  // past the row's end re-read its last chunk and are dropped)
  float4 v[NU], gv[NU], bv[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int ch = min(lane + 64 * u, nc - 1);
    v[u] = xr[ch];
    gv[u] = w4[ch];
    bv[u] = b4[ch];
  }
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    if (lane + 64 * u >= nc) v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    sum += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  const float mean = wave_sum_dpp(sum) / (float)d;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    if (lane + 64 * u < nc) {
      const float a = v[u].x - mean, bb = v[u].y - mean, cc = v[u].z - mean, dd = v[u].w - mean;
      sq += (a * a + bb * bb) + (cc * cc + dd * dd);
    }
  }
  const float var = wave_sum_dpp(sq) / (float)d;
  const float inv_std = 1.0f / sqrtf(var + eps);
  float4* orow = reinterpret_cast<float4*>(out + (size_t)row * d);
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int ch = lane + 64 * u;
    if (ch < nc) {
      const float4 g = gv[u], bi = bv[u];
      orow[ch] = make_float4((v[u].x - mean) * inv_std * g.x + bi.x, (v[u].y - mean) * inv_std * g.y + bi.y,
                             (v[u].z - mean) * inv_std * g.z + bi.z, (v[u].w - mean) * inv_std * g.w + bi.w);
    }
  }
}

void launch_layernorm(hipStream_t s, const float* x, const float* w, const float* b, float eps, int rows, int d,
                      float* out) {
  if (d % 4 == 0 && d <= 256 * LNW_MAXC) {
    const dim3 grid((rows + 3) / 4);
    switch ((d + 255) / 256) {
      case 1: layernorm_wave_kernel<1><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 2: layernorm_wave_kernel<2><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 3: layernorm_wave_kernel<3><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 4: layernorm_wave_kernel<4><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 5: layernorm_wave_kernel<5><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 6: layernorm_wave_kernel<6><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      case 7: layernorm_wave_kernel<7><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
      default: layernorm_wave_kernel<8><<<grid, 256, 0, s>>>(x, w, b, eps, rows, d, out); break;
    }
  } else
    layernorm_kernel<<<rows, 256, 0, s>>>(x, w, b, eps, d, out);
}

// ---------------------------------------------------------------------------
// Decode GEMV: one wave computes R output rows for up to BM sequences. Rows of
// W^T are contiguous, so each lane streams 16-byte vectors of a row
// (coalesced 1 KiB per wave instruction) and the wave reduces at the end.
// conv1d_forward, gpt2.rs:628-633 (matmul + add_broadcast), with the
// epilogues of forward_layer_cached (gpt2.rs:493-537).
// ---------------------------------------------------------------------------

struct GemvOut {
  float* y;
  int ldy;
  int epi;
  // QKV mode (q != nullptr): columns [0,d) -> q, [d,2d) -> K cache, [2d,3d) -> V cache.
  float* q;
  int ldq;
  int d;
  KvDst kv;
  const int* pos_dev;
};

// QKV epilogue of a decode step (q != nullptr): columns [0, d) are q, written
// to q[m][n]; [d, 3d) are the new token's k / v of sequence m, written into
// the cache at position *pos_dev (LayerKVCache::append, gpt2.rs:500-514).
struct SkinnyQkv {
  float* q;
  int ldq;
  int d;
  KvDst kv;
  const int* pos_dev;
};

// Skinny MFMA GEMM (defined with the prefill GEMM below); false when the
// shape does not suit it. With a workspace (ws) it may split k; kv_pre set
// (a prompt's c_attn) requires that split, whose reduction then writes the
// k / v columns into the cache (false otherwise).
static bool launch_skinny(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias,
                          float* C, long ldc, int M, int N, int K, int epi, const SkinnyQkv& qkv,
                          float* ws = nullptr, size_t ws_floats = 0, KvDst kv_pre = KvDst{}, int kv_T = 1,
                          int kv_past = 0);

template <int BM, int WT, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const void* __restrict__ W, const float* __restrict__ bias,
                                                   const float* __restrict__ x, int ldx, int nb, int N, int K,
                                                   GemvOut o) {
  constexpr int E = WVec<WT>::E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  if (row0 >= N) return;
  float acc[R][BM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BM; ++b) acc[r][b] = 0.f;

  for (int k = lane * E; k < K; k += 64 * E) {
    float xv[BM][E];
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      if (b < nb) {
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          float4 t = *reinterpret_cast<const float4*>(x + (size_t)b * ldx + k + e);
          xv[b][e] = t.x; xv[b][e + 1] = t.y; xv[b][e + 2] = t.z; xv[b][e + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) xv[b][e] = 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < N) {
        float wv[E];
        WVec<WT>::load(W, (size_t)(row0 + r) * K + k, wv);
#pragma unroll
        for (int b = 0; b < BM; ++b)
#pragma unroll
          for (int e = 0; e < E; ++e) acc[r][b] = fmaf(wv[e], xv[b][e], acc[r][b]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < BM; ++b) acc[r][b] = wave_sum(acc[r][b]);

  // Lane (r * BM + b) writes output (row0 + r, b); R * BM <= 64.
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int b = 0; b < BM; ++b) {
      const int n = row0 + r;
      if (lane == r * BM + b && n < N && b < nb) {
        float v = acc[r][b];
        if (o.q) {
          v = v + bias[n];
          const int d = o.d;
          if (n < d) {
            o.q[(size_t)b * o.ldq + n] = v;
          } else {
            const int c = n - (n < 2 * d ? d : 2 * d);
            const int hd = d / o.kv.n_head;
            const int h = c / hd, dd = c - h * hd;
            float* base = n < 2 * d ? o.kv.k : o.kv.v;
            const size_t off = (((size_t)b * o.kv.n_head + h) * o.kv.n_pos + *o.pos_dev) * hd + dd;
            base[off] = v;
          }
        } else {
          float* yp = o.y + (size_t)b * o.ldy + n;
          if (o.epi == EPI_BIAS) *yp = v + bias[n];
          else if (o.epi == EPI_BIAS_GELU) *yp = gelu_new(v + bias[n]);
          else if (o.epi == EPI_BIAS_RESID) *yp = *yp + (v + bias[n]);
          else *yp = v;
        }
      }
    }
  }
}

template <int BM, int WT>
static void gemv_dispatch_r(hipStream_t s, const void* W, const float* bias, const float* x, int ldx, int nb, int N,
                            int K, const GemvOut& o) {
  // Four rows per wave once there are plenty of rows (LM head), else one.
  if (N >= 16384 && BM <= 8) {
    constexpr int R = 4;
    const int waves = (N + R - 1) / R;
    gemv_kernel<BM, WT, R><<<(waves + 3) / 4, 256, 0, s>>>(W, bias, x, ldx, nb, N, K, o);
  } else {
    const int waves = N;
    gemv_kernel<BM, WT, 1><<<(waves + 3) / 4, 256, 0, s>>>(W, bias, x, ldx, nb, N, K, o);
  }
}

// A launch covers at most 16 sequences (BM); larger batches run as slices of
// 16 with x, the outputs and the cache rows offset to the slice's first
// sequence.
template <int WT>
static void gemv_dispatch_b(hipStream_t s, int nb, const void* W, const float* bias, const float* x, int ldx, int N,
                            int K, const GemvOut& o) {
  for (int b0 = 0; b0 < nb; b0 += 16) {
    const int n = nb - b0 < 16 ? nb - b0 : 16;
    GemvOut so = o;
    if (so.y) so.y += (size_t)b0 * so.ldy;
    if (so.q) {
      so.q += (size_t)b0 * so.ldq;
      const size_t seq = (size_t)so.kv.n_head * so.kv.n_pos * (so.d / so.kv.n_head);
      so.kv.k += b0 * seq;
      so.kv.v += b0 * seq;
    }
    const float* sx = x + (size_t)b0 * ldx;
    if (n <= 1) gemv_dispatch_r<1, WT>(s, W, bias, sx, ldx, n, N, K, so);
    else if (n <= 2) gemv_dispatch_r<2, WT>(s, W, bias, sx, ldx, n, N, K, so);
    else if (n <= 4) gemv_dispatch_r<4, WT>(s, W, bias, sx, ldx, n, N, K, so);
    else if (n <= 8) gemv_dispatch_r<8, WT>(s, W, bias, sx, ldx, n, N, K, so);
    else gemv_dispatch_r<16, WT>(s, W, bias, sx, ldx, n, N, K, so);
  }
}

void launch_gemv(hipStream_t s, int B, const void* W, int wtype, const float* bias, const float* x, int ldx,
                 float* y, int ldy, int N, int K, int epi) {
  // several sequences: MFMA reads each weight once for all of them
  if (B >= 2 && launch_skinny(s, x, ldx, W, wtype, bias, y, ldy, B, N, K, epi, SkinnyQkv{})) return;
  GemvOut o{};
  o.y = y; o.ldy = ldy; o.epi = epi;
  if (wtype == W_F32) gemv_dispatch_b<W_F32>(s, B, W, bias, x, ldx, N, K, o);
  else gemv_dispatch_b<W_BF16>(s, B, W, bias, x, ldx, N, K, o);
}

void launch_gemv_qkv(hipStream_t s, int B, const void* W, int wtype, const float* bias, const float* x, int ldx,
                     float* q, int ldq, int d, KvDst kv, const int* pos_dev) {
  if (B >= 2 && launch_skinny(s, x, ldx, W, wtype, bias, nullptr, 0, B, 3 * d, d, EPI_BIAS,
                              SkinnyQkv{q, ldq, d, kv, pos_dev}))
    return;
  GemvOut o{};
  o.q = q; o.ldq = ldq; o.d = d; o.kv = kv; o.pos_dev = pos_dev;
  if (wtype == W_F32) gemv_dispatch_b<W_F32>(s, B, W, bias, x, ldx, 3 * d, d, o);
  else gemv_dispatch_b<W_BF16>(s, B, W, bias, x, ldx, 3 * d, d, o);
}

// ---------------------------------------------------------------------------
// Decode attention, multi_head_attention_cached (gpt2.rs:772-834) for one new
// token per sequence: one block per (head, sequence). Scores live in LDS; the
// softmax is max / exp / sum / divide as in the reference, then P @ V.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void attn_decode_kernel(const float* __restrict__ q, int ldq,
                                                          const float* __restrict__ kc, const float* __restrict__ vc,
                                                          int H, int P, int hd, const int* __restrict__ pos_dev,
                                                          float* __restrict__ out, int ldo, int out_tk) {
  extern __shared__ float sm[];
  float* qs = sm;          // [hd]
  float* red = sm + 64;    // [16] block reduction scratch
  float* pv = sm + 80;     // [4][64]
  float* sc = sm + 336;    // [P]
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int len = *pos_dev + 1;
  const size_t head_off = ((size_t)b * H + h) * P * hd;
  const float* Kh = kc + head_off;
  const float* Vh = vc + head_off;
  if (tid < hd) qs[tid] = q[(size_t)b * ldq + h * hd + tid];
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int j = tid; j < len; j += blockDim.x) {
    float dot = 0.f;
    for (int dd = 0; dd < hd; ++dd) dot = fmaf(qs[dd], Kh[(size_t)j * hd + dd], dot);
    const float sv = dot * scale;
    sc[j] = sv;
    mx = fmaxf(mx, sv);
  }
  mx = block_reduce<true>(mx, red);
  float sum = 0.f;
  for (int j = tid; j < len; j += blockDim.x) {
    const float e = expf(sc[j] - mx);
    sc[j] = e;
    sum += e;
  }
  sum = block_reduce<false>(sum, red);
  for (int j = tid; j < len; j += blockDim.x) sc[j] = sc[j] / sum;
  __syncthreads();
  const int dd = tid & 63, part = tid >> 6;
  float acc = 0.f;
  if (dd < hd)
    for (int j = part; j < len; j += 4) acc = fmaf(sc[j], Vh[(size_t)j * hd + dd], acc);
  pv[part * 64 + dd] = acc;
  __syncthreads();
  if (tid < hd) {
    const size_t oi = out_tk ? xt_index(b, h * hd + tid, gridDim.y, out_tk) : (size_t)b * ldo + h * hd + tid;
    out[oi] = (pv[tid] + pv[64 + tid]) + (pv[128 + tid] + pv[192 + tid]);
  }
}

// Decode attention for head_dim 64 in one kernel: block (h, b) of NWV waves
// runs attn_item (attn_core.h).
template <int NWV>
__global__ __launch_bounds__(64 * NWV) void attn_decode_fused_kernel(const float* __restrict__ q, int ldq,
                                                                    const float* __restrict__ kc,
                                                                    const float* __restrict__ vc, int H, int P,
                                                                    const int* __restrict__ pos_dev,
                                                                    float* __restrict__ out, int ldo, int out_tk) {
  __shared__ float wp[NWV][AD_ITEM];
  attn_item<NWV>(q, ldq, kc, vc, H, P, *pos_dev + 1, blockIdx.x, blockIdx.y, out, ldo, out_tk, gridDim.y, wp);
}

void launch_attn_decode(hipStream_t s, int B, const float* q, int ldq, const float* kc, const float* vc, int n_head,
                        int n_pos, const int* pos_dev, float* out, int ldo, int out_tk) {
  // head_dim = ldq-independent: derived by the caller into n_head via ldo.
  const int hd = ldo / n_head;
  if (hd == 64) {
    // 16 waves per (head, sequence) while there are fewer pairs than CUs
    if (n_head * B < 256)
      attn_decode_fused_kernel<16>
          <<<dim3(n_head, B), 1024, 0, s>>>(q, ldq, kc, vc, n_head, n_pos, pos_dev, out, ldo, out_tk);
    else
      attn_decode_fused_kernel<8>
          <<<dim3(n_head, B), 512, 0, s>>>(q, ldq, kc, vc, n_head, n_pos, pos_dev, out, ldo, out_tk);
    return;
  }

  const size_t smem = (336 + (size_t)n_pos) * sizeof(float);
  attn_decode_kernel<<<dim3(n_head, B), 256, smem, s>>>(q, ldq, kc, vc, n_head, n_pos, hd, pos_dev, out, ldo,
                                                        out_tk);
}

// ---------------------------------------------------------------------------
// Argmax (argmax_f32, gpt2.rs:858-868): strict '>' from -inf, first index wins,
// NaN never wins, -0.0 ties with +0.0. Packed keys (argmax_key.h) reduced with
// a 64-bit atomic max; key 0 (nothing > -inf) decodes to index 0.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, long ld, int V,
                                                     unsigned long long* keys) {
  __shared__ unsigned long long red[4];
  const int row = blockIdx.y;
  const float* p = logits + (size_t)row * ld;
  unsigned long long best = 0ull;
  // eight loads of a thread in flight at once (the packed keys make the
  // reduction order-free)
  const int stride = gridDim.x * blockDim.x;
  for (int j0 = blockIdx.x * blockDim.x + threadIdx.x; j0 < V; j0 += 8 * stride) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = j0 + u * stride < V ? p[j0 + u * stride] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + u * stride;
      const unsigned long long k = j < V ? argmax_key(v[u], (uint32_t)j) : 0ull;
      best = k > best ? k : best;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = red[w] > best ? red[w] : best;
    atomicMax(&keys[row], best);
  }
}

void launch_argmax(hipStream_t s, const float* logits, long ld, int rows, int V, unsigned long long* keys) {
  int blocks = (V + 4095) / 4096;
  if (blocks > 64) blocks = 64;
  argmax_kernel<<<dim3(blocks, rows), 256, 0, s>>>(logits, ld, V, keys);
}

// One block of 256 threads, striding over any number of sequences.
__global__ __launch_bounds__(256) void finalize_kernel(int B, unsigned long long* keys, uint32_t* token,
                                                       uint32_t* ids_out, int ld_ids, int* pos_dev, int* step_dev,
                                                       unsigned* epoch) {
  // the counters and the keys are read together (one round trip); thread 0
  // advances the counters once every thread has read *step_dev
  const int step = *step_dev;
  int pos = 0;
  unsigned ep = 0u;
  if (threadIdx.x == 0) {
    pos = *pos_dev;
    if (epoch) ep = *epoch;
  }
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const uint32_t t = argmax_key_index(keys[b]);
    token[b] = t;
    if (ids_out) ids_out[(size_t)b * ld_ids + step] = t;
    keys[b] = 0ull;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    *pos_dev = pos + 1;
    *step_dev = step + 1;
    if (epoch) *epoch = ep + 1u;
  }
}

void launch_finalize(hipStream_t s, int B, unsigned long long* keys, uint32_t* token, uint32_t* ids_out, int ld_ids,
                     int* pos_dev, int* step_dev, unsigned* epoch) {
  finalize_kernel<<<1, 256, 0, s>>>(B, keys, token, ids_out, ld_ids, pos_dev, step_dev, epoch);
}

__global__ __launch_bounds__(256) void keys_to_tokens_kernel(int B, unsigned long long* keys, uint32_t* token) {
  for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < B; b += gridDim.x * blockDim.x) {
    token[b] = argmax_key_index(keys[b]);
    keys[b] = 0ull;
  }
}

void launch_keys_to_tokens(hipStream_t s, int B, unsigned long long* keys, uint32_t* token) {
  keys_to_tokens_kernel<<<1, 256, 0, s>>>(B, keys, token);
}

__global__ __launch_bounds__(256) void reset_keys_kernel(int B, unsigned long long* keys) {
  for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < B; b += gridDim.x * blockDim.x) keys[b] = 0ull;
}

void launch_reset_keys(hipStream_t s, int B, unsigned long long* keys) { reset_keys_kernel<<<1, 256, 0, s>>>(B, keys); }

// ---------------------------------------------------------------------------
// Prefill GEMM on fp32 MFMA (v_mfma_f32_32x32x2f32):
//   C[M][N] = epi(A[M][K] . W[N][K]^T)
// 128x128 block tile, 4 waves in a 2x2 arrangement, each wave 64x64 = 2x2
// MFMA tiles; BK = 16 with LDS double buffering. LDS holds A and W tiles
// k-major ([k][m], [k][n]) so MFMA operand reads are conflict-free.
// Operand layout of v_mfma_f32_32x32x2f32: lane l supplies A[l%32][l/32] and
// B[l/32][l%32]; accumulator i of lane l is D[(i/4)*8 + (l/32)*4 + i%4][l%32].
// ---------------------------------------------------------------------------

typedef float floatx16 __attribute__((ext_vector_type(16)));

// (a k-tile of 32 was measured slower: 86 against 106 TF/s on the c4 shapes,
// its LDS footprint halving the workgroups per CU)
constexpr int GBM = 128, GBN = 128, GBK = 16, GPAD = 4;

template <int WT>
__global__ __launch_bounds__(256) void gemm_kernel(const float* __restrict__ A, int lda, const void* __restrict__ W,
                                                   const float* __restrict__ bias, float* __restrict__ C, long ldc,
                                                   int M, int N, int K, int epi, int ks, float* __restrict__ ws) {
  __shared__ float As[2][GBK][GBM + GPAD];
  __shared__ float Ws[2][GBK][GBN + GPAD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int m0 = blockIdx.y * GBM, n0 = blockIdx.x * GBN;

  // Global->LDS mapping: 128 rows x GBK k = 32 * GBK float4; thread t loads
  // rows (t / KC) + RPP * h at k offset (t % KC) * 4, KC = GBK / 4 chunks per
  // row, RPP = 256 / KC rows per pass, NPS = 128 / RPP passes.
  constexpr int KC = GBK / 4, RPP = 256 / KC, NPS = GBM / RPP;
  const int lr = tid / KC, lk = (tid % KC) * 4;
  float4 ra[NPS], rw[NPS];

  auto gload = [&](int k0) {
#pragma unroll
    for (int h = 0; h < NPS; ++h) {
      const int m = m0 + lr + h * RPP, n = n0 + lr + h * RPP, k = k0 + lk;
      float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vw = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < M) {
        if (k + 3 < K) {
          va = *reinterpret_cast<const float4*>(A + (size_t)m * lda + k);
        } else {
          float t[4] = {0.f, 0.f, 0.f, 0.f};
          for (int e = 0; e < 4; ++e)
            if (k + e < K) t[e] = A[(size_t)m * lda + k + e];
          va = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
      if (n < N) {
        if (k + 3 < K) {
          if (WT == W_F32) {
            vw = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + (size_t)n * K + k);
          } else {
            uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(W) + (size_t)n * K + k);
            vw = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                             __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
          }
        } else {
          float t[4] = {0.f, 0.f, 0.f, 0.f};
          for (int e = 0; e < 4; ++e)
            if (k + e < K) t[e] = load_w1(W, (size_t)n * K + k + e, WT);
          vw = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
      ra[h] = va;
      rw[h] = vw;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int h = 0; h < NPS; ++h) {
      const int r = lr + h * RPP;
      As[buf][lk + 0][r] = ra[h].x; As[buf][lk + 1][r] = ra[h].y;
      As[buf][lk + 2][r] = ra[h].z; As[buf][lk + 3][r] = ra[h].w;
      Ws[buf][lk + 0][r] = rw[h].x; Ws[buf][lk + 1][r] = rw[h].y;
      Ws[buf][lk + 2][r] = rw[h].z; Ws[buf][lk + 3][r] = rw[h].w;
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // with ks > 1 (K a multiple of 16 * ks) workgroup z = blockIdx.z sums the
  // k range [z K / ks, (z + 1) K / ks) and stores its raw tile to ws[z]
  const int nk = ks > 1 ? K / ks / GBK : (K + GBK - 1) / GBK;
  const int kbeg = ks > 1 ? (int)blockIdx.z * (K / ks) : 0;
  gload(kbeg);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload(kbeg + (kt + 1) * GBK);
#pragma unroll
    for (int kk = 0; kk < GBK; kk += 2) {
      const int kr = kk + (lane >> 5);
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[cur][kr][wm + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Ws[cur][kr][wn + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  if (ws != nullptr) {
    float* wz = ws + (size_t)blockIdx.z * M * N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + j * 32 + (lane & 31);
        if (n >= N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (m < M) wz[(size_t)m * N + n] = acc[i][j][e];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn + j * 32 + (lane & 31);
      if (n >= N) continue;
      const float bv = bias ? bias[n] : 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (m < M) {
          float* cp = C + (size_t)m * ldc + n;
          const float v = acc[i][j][e];
          if (epi == EPI_BIAS) *cp = v + bv;
          else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
          else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
          else *cp = v;
        }
      }
    }
  }
}

// Prefill GEMM for f32 weights, K % 64 == 0: the same 128x128 tile and MFMA
// arrangement, fed by LDS-direct loads (global_load_lds_dwordx4) through a
// GL_NS-stage LDS ring, so no registers hold tiles in flight and three k-tiles
// are in flight while one is computed.
// - A stage holds the A and W tiles as 8 + 8 groups of 16 rows x 16 k (1 KiB,
//   one load instruction each: lane i fills bytes [16i, 16i + 16) of its
//   group). Lane i loads row r = i / 4 of the group, 4-float chunk
//   c = (i % 4) ^ gl_swz(row): an XOR swizzle that makes the operand reads
//   below conflict-free.
// - k is permuted inside a tile: MFMA step s of lane half h (lane / 32) uses
//   k = 8h + s, so a lane reads its 8 values of a row with two ds_read_b128.
//   A and W use the same permutation, so the products are those of the plain
//   order (the sum is taken over all 16 k of the tile either way).
constexpr int GL_NS = 4;
__device__ __forceinline__ int gl_swz(int row) { return (row >> 2) & 3; }

// global_load_lds_dwordx4 written out, so that the compiler's wait-count pass
// does not tie later LDS reads to these loads (it waited for all of them
// before every fourth tile's reads); the kernel orders them itself with
// gl_wait_barrier. M0 carries the wave-uniform LDS address.
__device__ __forceinline__ void gl_dma16(const float* src, const float* lds_dst) {
  const unsigned m0v =
      __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const __attribute__((address_space(3))) float*)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0v) : "memory", "m0");
}
// Wait until at most N of this wave's vector memory operations are
// outstanding, then a workgroup barrier; memory accesses do not move across.
template <int N>
__device__ __forceinline__ void gl_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// One k-tile step of gemm_lds_kernel on stage ST. Each stage is its own LDS
// array and the loop is unrolled over the four stages, so every LDS address
// is a base plus an immediate offset (about 1% faster than one array indexed
// by kt % 4).
template <int ST>
__device__ __forceinline__ void gl_step(int kt, int nk, float (&lds)[2][GBM * 16], float (&nxt)[2][GBM * 16],
                                        const float* const (&asrc)[2], const float* const (&wsrc)[2], int wave,
                                        const int (&aoff)[2][2], const int (&woff)[2][2], floatx16 (&acc)[2][2]) {
  // tile kt has landed once at most the loads of the GL_NS - 2 later tiles
  // (4 instructions each) are still outstanding; after the barrier every
  // wave's loads of tile kt are in and no wave reads tile kt - 1 any more
  if (kt + GL_NS - 2 < nk) gl_wait_barrier<(GL_NS - 2) * 4>();
  else gl_wait_barrier<0>();
  if (kt + GL_NS - 1 < nk) {
    const int k = (kt + GL_NS - 1) * 16;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int g = 2 * wave + q;
      gl_dma16(asrc[q] + k, &nxt[0][g * 256]);
      gl_dma16(wsrc[q] + k, &nxt[1][g * 256]);
    }
  }
  float4 a[2][2], b[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      a[i][c] = *reinterpret_cast<const float4*>(&lds[0][aoff[i][c]]);
      b[i][c] = *reinterpret_cast<const float4*>(&lds[1][woff[i][c]]);
    }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float4& av = a[i][s >> 2];
        const float4& bv = b[j][s >> 2];
        const int e = s & 3;
        const float x = e == 0 ? av.x : e == 1 ? av.y : e == 2 ? av.z : av.w;
        const float y = e == 0 ? bv.x : e == 1 ? bv.y : e == 2 ? bv.z : bv.w;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i][j], 0, 0, 0);
      }
  }
}

// Epilogue of the 128x128 tile kernels: wave tile (wm, wn) of block (m0, n0)
// in acc[i][j] (32x32 blocks, MFMA output layout), to ws[z] as a raw partial
// tile when ws is set, else with the epilogue (bias, gelu, residual; with kv
// set, c_attn's k / v columns go into the cache at (sequence, head, past + t)).
template <int I = 2, int J = 2>
__device__ __forceinline__ void gl_epilogue(const floatx16 (&acc)[I][J], int lane, int m0, int n0, int wm, int wn,
                                            int z, const float* __restrict__ bias, float* __restrict__ C, long ldc,
                                            int M, int N, int epi, const KvDst& kv, int kv_T, int kv_past,
                                            float* __restrict__ ws) {
  if (ws != nullptr) {
    float* wz = ws + (size_t)z * M * N;
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int n = n0 + wn + j * 32 + (lane & 31);
        if (n >= N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (m < M) wz[(size_t)m * N + n] = acc[i][j][e];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < I; ++i) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int n = n0 + wn + j * 32 + (lane & 31);
      if (n >= N) continue;
      const float bv = bias ? bias[n] : 0.f;
      if (kv.k != nullptr && n >= kv.d) {
        // k / v column of c_attn: into the cache at (sequence, head, past + t)
        const int which = n >= 2 * kv.d, cc = n - kv.d - which * kv.d;
        float* base = (which ? kv.v : kv.k) + (size_t)(cc >> 6) * kv.n_pos * 64 + (cc & 63);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (m < M) {
            const int sq = m / kv_T, t = m - sq * kv_T;
            base[((size_t)sq * kv.n_head * kv.n_pos + kv_past + t) * 64] = acc[i][j][e] + bv;
          }
        }
        continue;
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (m < M) {
          float* cp = C + (size_t)m * ldc + n;
          const float v = acc[i][j][e];
          if (epi == EPI_BIAS) *cp = v + bv;
          else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
          else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
          else *cp = v;
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void gemm_lds_kernel(const float* __restrict__ A, int lda,
                                                       const float* __restrict__ W, const float* __restrict__ bias,
                                                       float* __restrict__ C, long ldc, int M, int N, int K, int epi,
                                                       int m_fast, KvDst kv, int kv_T, int kv_past, int ks,
                                                       float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) float st0[2][GBM * 16];
  __shared__ __attribute__((aligned(16))) float st1[2][GBM * 16];
  __shared__ __attribute__((aligned(16))) float st2[2][GBM * 16];
  __shared__ __attribute__((aligned(16))) float st3[2][GBM * 16];
  static_assert(GL_NS == 4, "four stage arrays");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  // block order: with m_fast the row blocks of one W column block are
  // consecutive (W read once while A cycles through the cache), else the
  // column blocks of one A row block (A read once while W cycles)
  // with ks > 1 the k range is split: block b handles tile b % (nmb * nnb)
  // over k-split z = b / (nmb * nnb) and stores its raw partial tile to
  // ws[z] (summed and finished by splitk_reduce_kernel)
  const int nmb = (M + GBM - 1) / GBM, nnb = (N + GBN - 1) / GBN;
  const int bid = blockIdx.x % (nmb * nnb), z = blockIdx.x / (nmb * nnb);
  const int m0 = (m_fast ? bid % nmb : bid / nnb) * GBM, n0 = (m_fast ? bid / nmb : bid % nnb) * GBN;
  const int nk = K / 16 / ks;  // k-tiles of this split, a multiple of GL_NS

  // this lane's load sources: groups 2*wave and 2*wave + 1 of A and of W
  const int lr = lane >> 2;
  const float* asrc[2];
  const float* wsrc[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = (2 * wave + q) * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    asrc[q] = A + (size_t)min(m0 + row, M - 1) * lda + c * 4 + (size_t)z * nk * 16;
    wsrc[q] = W + (size_t)min(n0 + row, N - 1) * K + c * 4 + (size_t)z * nk * 16;
  }
  auto issue = [&](int kt, float (&st)[2][GBM * 16]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int g = 2 * wave + q;
      gl_dma16(asrc[q] + kt * 16, &st[0][g * 256]);
      gl_dma16(wsrc[q] + kt * 16, &st[1][g * 256]);
    }
  };

  // operand read offsets (floats within a stage's A or W tile): rows
  // wm + 32i + lane % 32 (A) and wn + 32j + lane % 32 (W), chunks 2h, 2h + 1
  const int h = lane >> 5;
  int aoff[2][2], woff[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ra = wm + 32 * i + (lane & 31), rw = wn + 32 * i + (lane & 31);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      aoff[i][c] = ra * 16 + (((2 * h + c) ^ gl_swz(ra)) * 4);
      woff[i][c] = rw * 16 + (((2 * h + c) ^ gl_swz(rw)) * 4);
    }
  }

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  issue(0, st0);
  issue(1, st1);
  issue(2, st2);
  for (int kt = 0; kt < nk; kt += GL_NS) {
    gl_step<0>(kt, nk, st0, st3, asrc, wsrc, wave, aoff, woff, acc);
    gl_step<1>(kt + 1, nk, st1, st0, asrc, wsrc, wave, aoff, woff, acc);
    gl_step<2>(kt + 2, nk, st2, st1, asrc, wsrc, wave, aoff, woff, acc);
    gl_step<3>(kt + 3, nk, st3, st2, asrc, wsrc, wave, aoff, woff, acc);
  }

  gl_epilogue(acc, lane, m0, n0, wm, wn, z, bias, C, ldc, M, N, epi, kv, kv_T, kv_past, ws);
}

// gemm_lds_kernel with 64 x 128 workgroup tiles (each wave 32 x 64, one A
// group of 16 rows and two W groups per stage), for f32 GEMMs of at most 1024
// rows: twice the workgroups of the 128 x 128 tiles, so fewer k splits and
// reductions (c3's 512-row and c2's 1024-row prefill GEMMs: 5-25% faster
// each, the split-k reduction included).
constexpr int G64M = 64;
template <int ST>
__device__ __forceinline__ void g64_step(int kt, int nk, float (&la)[G64M * 16], float (&lw)[GBN * 16],
                                         float (&na)[G64M * 16], float (&nw)[GBN * 16], const float* asrc,
                                         const float* const (&wsrc)[2], int wave, const int (&aoff)[2],
                                         const int (&woff)[2][2], floatx16 (&acc)[1][2]) {
  if (kt + GL_NS - 2 < nk) gl_wait_barrier<(GL_NS - 2) * 3>();
  else gl_wait_barrier<0>();
  if (kt + GL_NS - 1 < nk) {
    const int k = (kt + GL_NS - 1) * 16;
    gl_dma16(asrc + k, &na[wave * 256]);
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(wsrc[q] + k, &nw[(2 * wave + q) * 256]);
  }
  float4 a[2], b[2][2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    a[c] = *reinterpret_cast<const float4*>(&la[aoff[c]]);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j][c] = *reinterpret_cast<const float4*>(&lw[woff[j][c]]);
  }
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const float4& av = a[st >> 2];
    const int e = st & 3;
    const float x = e == 0 ? av.x : e == 1 ? av.y : e == 2 ? av.z : av.w;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float4& bv = b[j][st >> 2];
      const float y = e == 0 ? bv.x : e == 1 ? bv.y : e == 2 ? bv.z : bv.w;
      acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[0][j], 0, 0, 0);
    }
  }
}

__global__ __launch_bounds__(256) void gemm_lds64_kernel(const float* __restrict__ A, int lda,
                                                         const float* __restrict__ W, const float* __restrict__ bias,
                                                         float* __restrict__ C, long ldc, int M, int N, int K, int epi,
                                                         int m_fast, KvDst kv, int kv_T, int kv_past, int ks,
                                                         float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) float a0[G64M * 16], a1[G64M * 16], a2[G64M * 16], a3[G64M * 16];
  __shared__ __attribute__((aligned(16))) float w0[GBN * 16], w1[GBN * 16], w2[GBN * 16], w3[GBN * 16];
  static_assert(GL_NS == 4, "four stage arrays");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 64;
  const int nmb = (M + G64M - 1) / G64M, nnb = (N + GBN - 1) / GBN;
  const int bid = blockIdx.x % (nmb * nnb), z = blockIdx.x / (nmb * nnb);
  const int m0 = (m_fast ? bid % nmb : bid / nnb) * G64M, n0 = (m_fast ? bid / nmb : bid % nnb) * GBN;
  const int nk = K / 16 / ks;
  const int lr = lane >> 2;
  const float* asrc;
  {
    const int row = wave * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    asrc = A + (size_t)min(m0 + row, M - 1) * lda + c * 4 + (size_t)z * nk * 16;
  }
  const float* wsrc[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = (2 * wave + q) * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    wsrc[q] = W + (size_t)min(n0 + row, N - 1) * K + c * 4 + (size_t)z * nk * 16;
  }
  auto issue = [&](int kt, float (&la)[G64M * 16], float (&lw)[GBN * 16]) {
    gl_dma16(asrc + kt * 16, &la[wave * 256]);
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(wsrc[q] + kt * 16, &lw[(2 * wave + q) * 256]);
  };
  const int h = lane >> 5;
  int aoff[2], woff[2][2];
  {
    const int ra = wm + (lane & 31);
#pragma unroll
    for (int c = 0; c < 2; ++c) aoff[c] = ra * 16 + (((2 * h + c) ^ gl_swz(ra)) * 4);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rw = wn + 32 * j + (lane & 31);
#pragma unroll
      for (int c = 0; c < 2; ++c) woff[j][c] = rw * 16 + (((2 * h + c) ^ gl_swz(rw)) * 4);
    }
  }
  floatx16 acc[1][2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[0][j][e] = 0.f;
  issue(0, a0, w0);
  issue(1, a1, w1);
  issue(2, a2, w2);
  for (int kt = 0; kt < nk; kt += GL_NS) {
    g64_step<0>(kt, nk, a0, w0, a3, w3, asrc, wsrc, wave, aoff, woff, acc);
    g64_step<1>(kt + 1, nk, a1, w1, a0, w0, asrc, wsrc, wave, aoff, woff, acc);
    g64_step<2>(kt + 2, nk, a2, w2, a1, w1, asrc, wsrc, wave, aoff, woff, acc);
    g64_step<3>(kt + 3, nk, a3, w3, a2, w2, asrc, wsrc, wave, aoff, woff, acc);
  }
  gl_epilogue<1, 2>(acc, lane, m0, n0, wm, wn, z, bias, C, ldc, M, N, epi, kv, kv_T, kv_past, ws);
}

// gemm_lds_kernel for bf16 weights (the f32 activations times W stored as
// bf16, gpt2.rs Conv1D with bf16-rounded weights upcast in the product): the
// same 128x128 tiles, k-tiles of 16 and LDS-direct stage ring, with W's tile
// as 128 rows of 32 bytes (one load instruction per wave: lane i fills row
// 32 * wave + i / 2, 16-byte chunk (i % 2) ^ ((row >> 3) & 1)). Each lane's 8
// A values of a 32-row block enter v_mfma_f32_32x32x16_bf16 as three exact
// bf16 parts (split3), so every product is exact in f32 and the MFMA
// accumulates in f32: the f32 GEMM up to summation order, at the bf16 rate.
// Lane l holds A[row l % 32][k 8 (l / 32) .. + 8) and W[col l % 32][the same
// k] of a tile, the A reads of gemm_lds_kernel.
template <int ST>
__device__ __forceinline__ void glb_step(int kt, int nk, float (&la)[GBM * 16], float (&lw)[GBM * 8],
                                         float (&na)[GBM * 16], float (&nw)[GBM * 8], const float* const (&asrc)[2],
                                         const uint16_t* wsrc, int wave, const int (&aoff)[2][2], const int (&woff)[2],
                                         floatx16 (&acc)[2][2]) {
  // tile kt has landed once at most the loads of the GL_NS - 2 later tiles
  // (3 instructions each) are outstanding
  if (kt + GL_NS - 2 < nk) gl_wait_barrier<(GL_NS - 2) * 3>();
  else gl_wait_barrier<0>();
  if (kt + GL_NS - 1 < nk) {
    const int k = (kt + GL_NS - 1) * 16;
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(asrc[q] + k, &na[(2 * wave + q) * 256]);
    gl_dma16(reinterpret_cast<const float*>(wsrc + k), &nw[wave * 256]);
  }
  u4v b[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const u4v*>(&lw[woff[j]]);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 a0 = *reinterpret_cast<const float4*>(&la[aoff[i][0]]);
    const float4 a1 = *reinterpret_cast<const float4*>(&la[aoff[i][1]]);
    const float xs[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    u4v xh, xm, xl;
    split3(xs, xh, xm, xl);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x8 wb = as_bf16x8(b[j]);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xh), wb, acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xm), wb, acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xl), wb, acc[i][j], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ int glb_swz(int row) { return (row >> 3) & 1; }

__global__ __launch_bounds__(256) void gemm_lds_bf16_kernel(const float* __restrict__ A, int lda,
                                                            const uint16_t* __restrict__ W,
                                                            const float* __restrict__ bias, float* __restrict__ C,
                                                            long ldc, int M, int N, int K, int epi, int m_fast,
                                                            KvDst kv, int kv_T, int kv_past, int ks,
                                                            float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) float a0[GBM * 16], a1[GBM * 16], a2[GBM * 16], a3[GBM * 16];
  __shared__ __attribute__((aligned(16))) float w0[GBM * 8], w1[GBM * 8], w2[GBM * 8], w3[GBM * 8];
  static_assert(GL_NS == 4, "four stage arrays");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int nmb = (M + GBM - 1) / GBM, nnb = (N + GBN - 1) / GBN;
  const int bid = blockIdx.x % (nmb * nnb), z = blockIdx.x / (nmb * nnb);
  const int m0 = (m_fast ? bid % nmb : bid / nnb) * GBM, n0 = (m_fast ? bid / nmb : bid % nnb) * GBN;
  const int nk = K / 16 / ks;  // k-tiles of this split, a multiple of GL_NS

  // load sources: A groups 2*wave and 2*wave + 1 (as gemm_lds_kernel), W rows
  // 32*wave + lane / 2
  const int lr = lane >> 2;
  const float* asrc[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = (2 * wave + q) * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    asrc[q] = A + (size_t)min(m0 + row, M - 1) * lda + c * 4 + (size_t)z * nk * 16;
  }
  const uint16_t* wsrc;
  {
    const int row = 32 * wave + (lane >> 1);
    const int c = (lane & 1) ^ glb_swz(row);
    wsrc = W + (size_t)min(n0 + row, N - 1) * K + c * 8 + (size_t)z * nk * 16;
  }
  auto issue = [&](int kt, float (&la)[GBM * 16], float (&lw)[GBM * 8]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(asrc[q] + kt * 16, &la[(2 * wave + q) * 256]);
    gl_dma16(reinterpret_cast<const float*>(wsrc + kt * 16), &lw[wave * 256]);
  };
  // operand reads: A rows wm + 32i + lane % 32, chunks 2h and 2h + 1 (floats);
  // W rows wn + 32j + lane % 32, chunk h (8 bf16 = 4 floats' bytes)
  const int h = lane >> 5;
  int aoff[2][2], woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ra = wm + 32 * i + (lane & 31), rw = wn + 32 * i + (lane & 31);
#pragma unroll
    for (int c = 0; c < 2; ++c) aoff[i][c] = ra * 16 + (((2 * h + c) ^ gl_swz(ra)) * 4);
    woff[i] = rw * 8 + ((h ^ glb_swz(rw)) * 4);
  }

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  issue(0, a0, w0);
  issue(1, a1, w1);
  issue(2, a2, w2);
  for (int kt = 0; kt < nk; kt += GL_NS) {
    glb_step<0>(kt, nk, a0, w0, a3, w3, asrc, wsrc, wave, aoff, woff, acc);
    glb_step<1>(kt + 1, nk, a1, w1, a0, w0, asrc, wsrc, wave, aoff, woff, acc);
    glb_step<2>(kt + 2, nk, a2, w2, a1, w1, asrc, wsrc, wave, aoff, woff, acc);
    glb_step<3>(kt + 3, nk, a3, w3, a2, w2, asrc, wsrc, wave, aoff, woff, acc);
  }
  gl_epilogue(acc, lane, m0, n0, wm, wn, z, bias, C, ldc, M, N, epi, kv, kv_T, kv_past, ws);
}

// Skinny GEMM for few rows (a short prompt): the 128x128 tile kernel would
// launch only N/128 workgroups. Here a workgroup computes a 32x32 output tile
// and each of its 4 waves a quarter of K. Step e of a wave's MFMA chain pairs
// k = k0 + e (lanes 0-31) with k = k0 + KH + e (lanes 32-63), KH = half the
// wave's K range, so each lane reads two contiguous runs (row m of A from L2,
// row n of W streamed from HBM) as 16-byte vectors. The four partial tiles
// are summed in LDS in wave order; then the tile kernel's epilogues.
// Needs K % 64 == 0 (every GPT-2 width).
constexpr int SK_CHUNK = 8;  // k per lane-run per loop step

template <int WT>
__device__ __forceinline__ void load8(const void* W, size_t idx, float* out) {
  if (WT == W_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + idx);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + idx + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(W) + idx);
    out[0] = __uint_as_float(u.x << 16); out[1] = __uint_as_float(u.x & 0xffff0000u);
    out[2] = __uint_as_float(u.y << 16); out[3] = __uint_as_float(u.y & 0xffff0000u);
    out[4] = __uint_as_float(u.z << 16); out[5] = __uint_as_float(u.z & 0xffff0000u);
    out[6] = __uint_as_float(u.w << 16); out[7] = __uint_as_float(u.w & 0xffff0000u);
  }
}

template <int WT>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const float* __restrict__ A, int lda,
                                                          const void* __restrict__ W, const float* __restrict__ bias,
                                                          float* __restrict__ C, long ldc, int M, int N, int K,
                                                          int epi, SkinnyQkv qkv, int ks, float* __restrict__ ws) {
  __shared__ float red[4][32][33];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, hh = lane >> 5;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  // with ks > 1 workgroup z = blockIdx.z takes the k range [z K / ks,
  // (z + 1) K / ks) (a multiple of 64) and stores its raw tile to ws[z]
  const int KZ = K / ks, KW = KZ / 4, KH = KW / 2;
  const int k0 = (int)blockIdx.z * KZ + wave * KW + hh * KH;  // this lane's run: [k0, k0 + KH)
  const float* arow = A + (size_t)min(m0 + r, M - 1) * lda + k0;
  const size_t wrow = (size_t)min(n0 + r, N - 1) * K + k0;
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  // SK_DEPTH chunks in flight: chunk c lives in slot c % SK_DEPTH
  constexpr int SK_DEPTH = 4;
  const int nch = KH / SK_CHUNK;
  float a[SK_DEPTH][SK_CHUNK], w[SK_DEPTH][SK_CHUNK];
#pragma unroll
  for (int d = 0; d < SK_DEPTH; ++d) {
    const int k = min(d, nch - 1) * SK_CHUNK;
    load8<W_F32>(arow, k, a[d]);
    load8<WT>(W, wrow + k, w[d]);
  }
  for (int c0 = 0; c0 < nch; c0 += SK_DEPTH) {
#pragma unroll
    for (int d = 0; d < SK_DEPTH; ++d) {
      if (c0 + d < nch) {
#pragma unroll
        for (int e = 0; e < SK_CHUNK; ++e)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d][e], w[d][e], acc, 0, 0, 0);
      }
      const int kn = min(c0 + d + SK_DEPTH, nch - 1) * SK_CHUNK;  // refill (a repeat past the end)
      load8<W_F32>(arow, kn, a[d]);
      load8<WT>(W, wrow + kn, w[d]);
    }
  }
  // lane holds the wave's partial of C[m0 + (i/4)*8 + hh*4 + i%4][n0 + r]
#pragma unroll
  for (int i = 0; i < 16; ++i) red[wave][(i >> 2) * 8 + hh * 4 + (i & 3)][r] = acc[i];
  __syncthreads();
  for (int idx = tid; idx < 32 * 32; idx += 256) {
    const int mi = idx >> 5, ni = idx & 31;
    const int m = m0 + mi, n = n0 + ni;
    if (m >= M || n >= N) continue;
    const float v = ((red[0][mi][ni] + red[1][mi][ni]) + red[2][mi][ni]) + red[3][mi][ni];
    if (ws != nullptr) {
      ws[(size_t)blockIdx.z * M * N + (size_t)m * N + n] = v;
      continue;
    }
    const float bv = bias ? bias[n] : 0.f;
    if (qkv.q) {
      const int d = qkv.d;
      if (n < d) {
        qkv.q[(size_t)m * qkv.ldq + n] = v + bv;
      } else {
        const int cc = n - (n < 2 * d ? d : 2 * d);
        const int hd = d / qkv.kv.n_head;
        const int h = cc / hd, dd = cc - h * hd;
        float* base = n < 2 * d ? qkv.kv.k : qkv.kv.v;
        base[(((size_t)m * qkv.kv.n_head + h) * qkv.kv.n_pos + *qkv.pos_dev) * hd + dd] = v + bv;
      }
      continue;
    }
    float* cp = C + (size_t)m * ldc + n;
    if (epi == EPI_BIAS) *cp = v + bv;
    else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
    else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
    else *cp = v;
  }
}

// The same for at most 16 rows (a decode batch) on v_mfma_f32_16x16x4f32,
// whose 16-wide tiles waste less of the matrix unit on absent rows and give
// twice as many workgroups: lane l supplies A[l%16][l/16] and B[l/16][l%16]
// and holds D[(l/16)*4 + i][l%16] in accumulator i. Step e pairs the four
// k = k0 + q*KQ + e (q = l/16, KQ = a quarter of the wave's K range), so a
// lane again reads contiguous runs.
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int WT>
__device__ __forceinline__ void load4(const void* W, size_t idx, float* out) {
  if (WT == W_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(W) + idx);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(W) + idx);
    out[0] = __uint_as_float(u.x << 16); out[1] = __uint_as_float(u.x & 0xffff0000u);
    out[2] = __uint_as_float(u.y << 16); out[3] = __uint_as_float(u.y & 0xffff0000u);
  }
}

template <int WT, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_skinny16_kernel(const float* __restrict__ A, int lda,
                                                                const void* __restrict__ W,
                                                                const float* __restrict__ bias, float* __restrict__ C,
                                                                long ldc, int M, int N, int K, int epi, SkinnyQkv qkv) {
  __shared__ float red[NW][16][17];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, qq = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int KW = K / NW, KQ = KW / 4;
  const int k0 = wave * KW + qq * KQ;  // this lane's run: [k0, k0 + KQ)
  const float* arow = A + (size_t)min(r, M - 1) * lda + k0;
  const size_t wrow = (size_t)min(n0 + r, N - 1) * K + k0;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  constexpr int DEPTH = 4;
  const int nch = KQ / 4;
  float a[DEPTH][4], w[DEPTH][4];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    const int k = min(d, nch - 1) * 4;
    load4<W_F32>(arow, k, a[d]);
    load4<WT>(W, wrow + k, w[d]);
  }
  for (int c0 = 0; c0 < nch; c0 += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      if (c0 + d < nch) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[d][e], w[d][e], acc, 0, 0, 0);
      }
      const int kn = min(c0 + d + DEPTH, nch - 1) * 4;  // refill (a repeat past the end)
      load4<W_F32>(arow, kn, a[d]);
      load4<WT>(W, wrow + kn, w[d]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][qq * 4 + i][r] = acc[i];
  __syncthreads();
  if (tid < 256) {
    const int mi = tid >> 4, ni = tid & 15;
    const int m = mi, n = n0 + ni;
    if (m < M && n < N) {
      float v = red[0][mi][ni];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) v += red[ww][mi][ni];
      const float bv = bias ? bias[n] : 0.f;
      if (qkv.q) {
        const int d = qkv.d;
        if (n < d) {
          qkv.q[(size_t)m * qkv.ldq + n] = v + bv;
        } else {
          const int cc = n - (n < 2 * d ? d : 2 * d);
          const int hd = d / qkv.kv.n_head;
          const int h = cc / hd, dd = cc - h * hd;
          float* base = n < 2 * d ? qkv.kv.k : qkv.kv.v;
          base[(((size_t)m * qkv.kv.n_head + h) * qkv.kv.n_pos + *qkv.pos_dev) * hd + dd] = v + bv;
        }
      } else {
        float* cp = C + (size_t)m * ldc + n;
        if (epi == EPI_BIAS) *cp = v + bv;
        else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
        else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
        else *cp = v;
      }
    }
  }
}

// Prompt GEMM for 17..32 rows with f32 weights, K % 64 == 0: gemm_lds_kernel's
// LDS-direct ring (4 stages, XOR-swizzled 16-byte chunks, k permuted inside a
// tile) with a 32 x 128 tile: the 32 rows of A and 128 rows of W (output
// columns) per 16-k stage, wave w computing columns [32w, 32w + 32) with one
// v_mfma_f32_32x32x2f32 block. The weights stream as whole 64-byte row runs
// (four lanes per row), where gemm_skinny_kernel's register loads give each
// lane its own row (32 lines per wave instruction). Each wave loads two of
// the eight W groups and one A group (waves 2 and 3 repeat A's into a spare
// region, so that every wave issues the same three loads per stage).
// With ks > 1, column block b over k-split z = blockIdx.x / nnb stores its raw
// tile to ws[z] for splitk_reduce_kernel.
constexpr int SL_BN = 128;
constexpr int SL_STAGE = (4 + 8) * 256;  // floats per stage: A groups 0-1 (2-3 spare), W groups 0-7
template <int ST>
__device__ __forceinline__ void sl_step(int kt, int nk, float (&stg)[SL_STAGE], float (&nxt)[SL_STAGE],
                                        const float* asrc, const float* const (&wsrc)[2], int wave,
                                        const int (&aoff)[2], const int (&woff)[2], floatx16& acc) {
  // tile kt has landed once at most the loads of the GL_NS - 2 later tiles
  // (3 instructions each) are outstanding; after the barrier no wave reads
  // tile kt - 1 any more
  if (kt + GL_NS - 2 < nk) gl_wait_barrier<(GL_NS - 2) * 3>();
  else gl_wait_barrier<0>();
  if (kt + GL_NS - 1 < nk) {
    const int k = (kt + GL_NS - 1) * 16;
    gl_dma16(asrc + k, &nxt[wave * 256]);
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(wsrc[q] + k, &nxt[(4 + 2 * wave + q) * 256]);
  }
  float4 a[2], b[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    a[c] = *reinterpret_cast<const float4*>(&stg[aoff[c]]);
    b[c] = *reinterpret_cast<const float4*>(&stg[4 * 256 + woff[c]]);
  }
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const float4& av = a[st >> 2];
    const float4& bv = b[st >> 2];
    const int e = st & 3;
    const float x = e == 0 ? av.x : e == 1 ? av.y : e == 2 ? av.z : av.w;
    const float y = e == 0 ? bv.x : e == 1 ? bv.y : e == 2 ? bv.z : bv.w;
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc, 0, 0, 0);
  }
}

__global__ __launch_bounds__(256) void gemm_skinny_lds_kernel(const float* __restrict__ A, int lda,
                                                              const float* __restrict__ W,
                                                              const float* __restrict__ bias, float* __restrict__ C,
                                                              long ldc, int M, int N, int K, int epi, int ks,
                                                              float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) float st0[SL_STAGE];
  __shared__ __attribute__((aligned(16))) float st1[SL_STAGE];
  __shared__ __attribute__((aligned(16))) float st2[SL_STAGE];
  __shared__ __attribute__((aligned(16))) float st3[SL_STAGE];
  static_assert(GL_NS == 4, "four stage arrays");
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nnb = (N + SL_BN - 1) / SL_BN;
  const int n0 = (blockIdx.x % nnb) * SL_BN, z = blockIdx.x / nnb;
  const int nk = K / 16 / ks;  // k-tiles of this split, a multiple of GL_NS
  // load sources: A group wave & 1, W groups 2*wave and 2*wave + 1
  const int lr = lane >> 2;
  const float* asrc;
  const float* wsrc[2];
  {
    const int row = (wave & 1) * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    asrc = A + (size_t)min(row, M - 1) * lda + c * 4 + (size_t)z * nk * 16;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int row = (2 * wave + q) * 16 + lr;
    const int c = (lane & 3) ^ gl_swz(row);
    wsrc[q] = W + (size_t)min(n0 + row, N - 1) * K + c * 4 + (size_t)z * nk * 16;
  }
  auto issue = [&](int kt, float (&stg)[SL_STAGE]) {
    gl_dma16(asrc + kt * 16, &stg[wave * 256]);
#pragma unroll
    for (int q = 0; q < 2; ++q) gl_dma16(wsrc[q] + kt * 16, &stg[(4 + 2 * wave + q) * 256]);
  };
  // operand reads: A row lane % 32, W row 32*wave + lane % 32, chunks 2h, 2h + 1
  const int h = lane >> 5;
  int aoff[2], woff[2];
  {
    const int ra = lane & 31, rw = 32 * wave + (lane & 31);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      aoff[c] = ra * 16 + (((2 * h + c) ^ gl_swz(ra)) * 4);
      woff[c] = rw * 16 + (((2 * h + c) ^ gl_swz(rw)) * 4);
    }
  }
  floatx16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  issue(0, st0);
  issue(1, st1);
  issue(2, st2);
  for (int kt = 0; kt < nk; kt += GL_NS) {
    sl_step<0>(kt, nk, st0, st3, asrc, wsrc, wave, aoff, woff, acc);
    sl_step<1>(kt + 1, nk, st1, st0, asrc, wsrc, wave, aoff, woff, acc);
    sl_step<2>(kt + 2, nk, st2, st1, asrc, wsrc, wave, aoff, woff, acc);
    sl_step<3>(kt + 3, nk, st3, st2, asrc, wsrc, wave, aoff, woff, acc);
  }
  // lane holds C[(e / 4) * 8 + h * 4 + e % 4][n0 + 32 * wave + lane % 32]
  const int n = n0 + 32 * wave + (lane & 31);
  if (n >= N) return;
  if (ws != nullptr) {
    float* wz = ws + (size_t)z * M * N;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = (e >> 2) * 8 + h * 4 + (e & 3);
      if (m < M) wz[(size_t)m * N + n] = acc[e];
    }
    return;
  }
  const float bv = bias ? bias[n] : 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = (e >> 2) * 8 + h * 4 + (e & 3);
    if (m >= M) continue;
    float* cp = C + (size_t)m * ldc + n;
    const float v = acc[e];
    if (epi == EPI_BIAS) *cp = v + bv;
    else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
    else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
    else *cp = v;
  }
}

// k-splits of gemm_skinny_lds_kernel: 1 when its column blocks give >= 192
// workgroups, else the smallest split into whole 4-tile stages giving >= 240,
// or the largest such split up to 16 (c1's 32-token prefill: 0.72 ms with
// at most 16, 0.73 with 12, 0.75 with 8, 0.76 with up to 48, whose
// reductions read 48 partials per output).
static int skinny_lds_splitk_factor(int M, int N, int K) {
  const int tiles = (N + SL_BN - 1) / SL_BN;
  if (M > 32 || M <= 16 || K % 64 != 0 || tiles >= 192) return 1;
  const int nk = K / 16;
  int best = 1;
  for (int sp = 2; sp <= nk / GL_NS && sp <= 16; ++sp) {
    if ((nk / GL_NS) % sp != 0) continue;
    best = sp;
    if (tiles * sp >= 240) break;
  }
  return best;
}

// k-splits of gemm_skinny_kernel (rows M <= 64, 32 x 32 tiles): 1 when the
// tiles give >= 192 workgroups, else the smallest split of K into multiples
// of 64 giving >= 240, or the largest valid one up to 16.
static int skinny_splitk_factor(int M, int N, int K) {
  const int tiles = ((N + 31) / 32) * ((M + 31) / 32);
  if (M > 64 || M <= 16 || tiles >= 192 || K % 64 != 0) return 1;
  const int nk = K / 64;
  int best = 1;
  for (int sp = 2; sp <= 16; ++sp) {
    if (nk % sp != 0) continue;
    best = sp;
    if (tiles * sp >= 240) break;
  }
  return best;
}

static void splitk_reduce(hipStream_t s, const float* ws, int ks, int M, int N, const float* bias, float* C, long ldc,
                          int epi, KvDst kv, int kv_T, int kv_past);

static bool launch_skinny(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias,
                          float* C, long ldc, int M, int N, int K, int epi, const SkinnyQkv& qkv, float* ws,
                          size_t ws_floats, KvDst kv_pre, int kv_T, int kv_past) {
  if (M > 64 || K % 64 != 0 || lda % 4 != 0) return false;
  if (wtype == W_F32 && M > 16 && M <= 32 && qkv.q == nullptr && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(W) & 15) == 0) {
    int ks = skinny_lds_splitk_factor(M, N, K);
    if (ks > 1 && (ws == nullptr || (size_t)ks * M * N > ws_floats)) ks = 1;
    if (ks > 1 || kv_pre.k == nullptr) {
      const int nnb = (N + SL_BN - 1) / SL_BN;
      gemm_skinny_lds_kernel<<<nnb * ks, 256, 0, s>>>(A, lda, static_cast<const float*>(W), bias, C, ldc, M, N, K,
                                                      epi, ks, ks > 1 ? ws : nullptr);
      if (ks > 1) splitk_reduce(s, ws, ks, M, N, bias, C, ldc, epi, kv_pre, kv_T, kv_past);
      return true;
    }
  }
  int ks = qkv.q == nullptr ? skinny_splitk_factor(M, N, K) : 1;
  if (ks > 1 && (ws == nullptr || (size_t)ks * M * N > ws_floats)) ks = 1;
  if (ks > 1) {
    // partial tiles, then the fixed-order sum with the epilogue (and, for a
    // prompt's c_attn, its k / v columns written into the cache)
    dim3 grid((N + 31) / 32, (M + 31) / 32, ks);
    if (wtype == W_F32)
      gemm_skinny_kernel<W_F32><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv, ks, ws);
    else
      gemm_skinny_kernel<W_BF16><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv, ks, ws);
    splitk_reduce(s, ws, ks, M, N, bias, C, ldc, epi, kv_pre, kv_T, kv_past);
    return true;
  }
  if (kv_pre.k != nullptr) return false;  // the prompt's k / v columns need the separate append
  if (M <= 16) {
    // (8 waves with twice the loads in flight measured slower: each wave
    // instruction already touches 16 rows, the address units saturate)
    const dim3 grid((N + 15) / 16);
    if (wtype == W_F32)
      gemm_skinny16_kernel<W_F32, 4><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv);
    else
      gemm_skinny16_kernel<W_BF16, 4><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv);
    return true;
  }
  dim3 grid((N + 31) / 32, (M + 31) / 32);
  if (wtype == W_F32)
    gemm_skinny_kernel<W_F32><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv, 1, nullptr);
  else
    gemm_skinny_kernel<W_BF16><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, qkv, 1, nullptr);
  return true;
}

// Sum of the ks split-k partial tiles of gemm_lds_kernel (ws[z][m][n], in z
// order) and the epilogue that kernel applies without a split (bias, gelu,
// residual; with kv set, the k / v columns of c_attn go into the cache).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int ks, int M, int N,
                                                            const float* __restrict__ bias, float* __restrict__ C,
                                                            long ldc, int epi, KvDst kv, int kv_T, int kv_past) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * N) return;
  const int m = (int)(i / N), n = (int)(i - (long)m * N);
  // every partial of a chunk of 16 in flight at once (the splits never
  // exceed 16, so one round trip), summed in z order
  const size_t MN = (size_t)M * N;
  float v = 0.f;
  for (int z0 = 0; z0 < ks; z0 += 16) {
    float t[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) t[u] = z0 + u < ks ? ws[(size_t)(z0 + u) * MN + i] : 0.f;
    if (z0 == 0) v = t[0];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if ((z0 > 0 || u > 0) && z0 + u < ks) v += t[u];
  }
  const float bv = bias ? bias[n] : 0.f;
  if (kv.k != nullptr && n >= kv.d) {
    const int which = n >= 2 * kv.d, cc = n - kv.d - which * kv.d;
    const int sq = m / kv_T, t = m - sq * kv_T;
    float* base = which ? kv.v : kv.k;
    base[((size_t)sq * kv.n_head + (cc >> 6)) * kv.n_pos * 64 + (size_t)(kv_past + t) * 64 + (cc & 63)] = v + bv;
    return;
  }
  float* cp = C + (size_t)m * ldc + n;
  if (epi == EPI_BIAS) *cp = v + bv;
  else if (epi == EPI_BIAS_GELU) *cp = gelu_new(v + bv);
  else if (epi == EPI_BIAS_RESID) *cp = *cp + (v + bv);
  else *cp = v;
}

static void splitk_reduce(hipStream_t s, const float* ws, int ks, int M, int N, const float* bias, float* C, long ldc,
                          int epi, KvDst kv, int kv_T, int kv_past) {
  const long total = (long)M * N;
  splitk_reduce_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(ws, ks, M, N, bias, C, ldc, epi, kv, kv_T,
                                                                      kv_past);
}

// k-splits of gemm_lds_kernel for an M x N x K GEMM: 1 when the output tiles
// alone give enough workgroups (>= 192) or M < 128, else the smallest split
// that gives >= 240 workgroups (each split a multiple of 4 k-tiles), or the
// largest valid one up to 16. (Prefills of a few hundred rows otherwise run
// their d-wide GEMMs on 32-48 of the 256 CUs.)
// granule: k-tiles of 16 a split must hold a multiple of (GL_NS for
// gemm_lds_kernel's stage ring, 1 for gemm_kernel).
int gemm_splitk_factor(int M, int N, int K, int granule) {
  const int tiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
  if (M < 128 || tiles >= 192 || K % (16 * granule) != 0) return 1;
  const int nk = K / 16;
  int best = 1;
  for (int s = 2; s <= 16; ++s) {
    if (nk % (granule * s) != 0) continue;
    best = s;
    if (tiles * s >= 240) break;
  }
  return best;
}

// k-splits of gemm_lds64_kernel (M <= 1024): as gemm_splitk_factor, over its
// 64 x 128 output tiles (and, as there, none below 128 rows).
static int gemm64_splitk_factor(int M, int N, int K) {
  const int tiles = ((N + GBN - 1) / GBN) * ((M + G64M - 1) / G64M);
  if (M < 128 || M > 1024 || tiles >= 192 || K % (16 * GL_NS) != 0) return 1;
  const int nkt = K / 16;
  int best = 1;
  for (int sp = 2; sp <= 16; ++sp) {
    if (nkt % (GL_NS * sp) != 0) continue;
    best = sp;
    if (tiles * sp >= 240) break;
  }
  return best;
}

size_t gemm_splitk_ws_floats(int M, int N, int K) {
  // the largest of the kernels' needs (which one runs depends on the weight
  // type, the row count and alignment)
  const int ks = std::max(std::max(std::max(gemm_splitk_factor(M, N, K, GL_NS), gemm_splitk_factor(M, N, K, 1)),
                                   std::max(skinny_splitk_factor(M, N, K), skinny_lds_splitk_factor(M, N, K))),
                          gemm64_splitk_factor(M, N, K));
  return ks > 1 ? (size_t)ks * M * N : 0;
}

static bool gemm_lds_ok(const float* A, int lda, const void* W, int wtype, int K) {
  return K % 64 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(W) & 15) == 0;
}

// gemm_lds_kernel (f32 W) or gemm_lds_bf16_kernel (bf16 W), split over k
// when that fills the GPU and ws holds the partial tiles (ws_floats of them),
// then the split-k reduction.
static void launch_gemm_lds(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias,
                            float* C, long ldc, int M, int N, int K, int epi, KvDst kv, int kv_T, int kv_past,
                            float* ws, size_t ws_floats) {
  const int nb = ((N + GBN - 1) / GBN) * ((M + GBM - 1) / GBM);
  int ks = gemm_splitk_factor(M, N, K, GL_NS);
  if (ks > 1 && (ws == nullptr || (size_t)ks * M * N > ws_floats)) ks = 1;
  if (wtype == W_F32 && M <= 1024) {
    // 64 x 128 tiles (gemm_lds64_kernel)
    const int nb64 = ((N + GBN - 1) / GBN) * ((M + G64M - 1) / G64M);
    int ks64 = gemm64_splitk_factor(M, N, K);
    if (ks64 > 1 && (ws == nullptr || (size_t)ks64 * M * N > ws_floats)) ks64 = 1;
    gemm_lds64_kernel<<<nb64 * ks64, 256, 0, s>>>(A, lda, static_cast<const float*>(W), bias, C, ldc, M, N, K, epi,
                                                  N > M ? 1 : 0, kv, kv_T, kv_past, ks64, ks64 > 1 ? ws : nullptr);
    if (ks64 > 1) splitk_reduce(s, ws, ks64, M, N, bias, C, ldc, epi, kv, kv_T, kv_past);
    return;
  }
  float* wsk = ks > 1 ? ws : nullptr;
  if (wtype == W_F32)
    gemm_lds_kernel<<<nb * ks, 256, 0, s>>>(A, lda, static_cast<const float*>(W), bias, C, ldc, M, N, K, epi,
                                            N > M ? 1 : 0, kv, kv_T, kv_past, ks, wsk);
  else
    gemm_lds_bf16_kernel<<<nb * ks, 256, 0, s>>>(A, lda, static_cast<const uint16_t*>(W), bias, C, ldc, M, N, K,
                                                 epi, N > M ? 1 : 0, kv, kv_T, kv_past, ks, wsk);
  if (ks > 1) splitk_reduce(s, ws, ks, M, N, bias, C, ldc, epi, kv, kv_T, kv_past);
}

void launch_gemm(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias, float* C,
                 long ldc, int M, int N, int K, int epi, float* ws, size_t ws_floats) {
  if (launch_skinny(s, A, lda, W, wtype, bias, C, ldc, M, N, K, epi, SkinnyQkv{}, ws, ws_floats)) return;
  dim3 grid((N + GBN - 1) / GBN, (M + GBM - 1) / GBM);
  if (gemm_lds_ok(A, lda, W, wtype, K))
    // (256 x 128 tiles with 3 stages, bounded to two waves per SIMD, were 2-4%
    // faster on the c4 shapes without an epilogue but made the c4 prefill
    // slower, 70.7k against 72.5k tokens/s; 3 stages at three waves per SIMD
    // and 2 stages at four were no faster than this kernel)
    launch_gemm_lds(s, A, lda, W, wtype, bias, C, ldc, M, N, K, epi, KvDst{}, 1, 0, ws, ws_floats);
  else {
    int ks = gemm_splitk_factor(M, N, K, 1);
    if (ks > 1 && (ws == nullptr || (size_t)ks * M * N > ws_floats)) ks = 1;
    grid.z = ks;
    float* wsk = ks > 1 ? ws : nullptr;
    if (wtype == W_F32) gemm_kernel<W_F32><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, ks, wsk);
    else gemm_kernel<W_BF16><<<grid, 256, 0, s>>>(A, lda, W, bias, C, ldc, M, N, K, epi, ks, wsk);
    if (ks > 1) splitk_reduce(s, ws, ks, M, N, bias, C, ldc, epi, KvDst{}, 1, 0);
  }
}

void launch_gemm_qkv(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias, float* C,
                     long ldc, int M, int K, int S, int T, int past, KvDst kv, float* ws, size_t ws_floats) {
  const int N = 3 * kv.d;
  if (M > 64 && gemm_lds_ok(A, lda, W, wtype, K) && kv.d == 64 * kv.n_head) {
    launch_gemm_lds(s, A, lda, W, wtype, bias, C, ldc, M, N, K, EPI_BIAS, kv, T, past, ws, ws_floats);
    return;
  }
  // a prompt of at most 64 rows: the split skinny GEMM's reduction writes the
  // k / v columns into the cache itself
  if (launch_skinny(s, A, lda, W, wtype, bias, C, ldc, M, N, K, EPI_BIAS, SkinnyQkv{}, ws, ws_floats, kv, T, past))
    return;
  launch_gemm(s, A, lda, W, wtype, bias, C, ldc, M, N, K, EPI_BIAS, ws, ws_floats);
  launch_kv_append(s, C, S, T, past, kv);
}

// ---------------------------------------------------------------------------
// Prefill KV append (LayerKVCache::append with the per-head split of
// gpt2.rs:500-514): qkv rows [S*T][3d] -> cache positions past .. past+T-1.
// ---------------------------------------------------------------------------

__global__ void kv_append_kernel(const float* __restrict__ qkv, int T, int past, KvDst kv) {
  const int r = blockIdx.x;  // s * T + t
  const int sidx = r / T, t = r - sidx * T;
  const int d = kv.d, hd = d / kv.n_head;
  for (int c = threadIdx.x; c < 2 * d; c += blockDim.x) {
    const int which = c / d, cc = c - which * d;
    const int h = cc / hd, dd = cc - h * hd;
    const float v = qkv[(size_t)r * 3 * d + d + c];
    float* base = which == 0 ? kv.k : kv.v;
    base[(((size_t)sidx * kv.n_head + h) * kv.n_pos + past + t) * hd + dd] = v;
  }
}

void launch_kv_append(hipStream_t s, const float* qkv, int S, int T, int past, KvDst kv) {
  kv_append_kernel<<<S * T, 256, 0, s>>>(qkv, T, past, kv);
}

// ---------------------------------------------------------------------------
// Prefill causal attention (multi_head_attention_cached, gpt2.rs:772-834, for
// new_len > 1): one thread per query row, keys/values staged through LDS in
// tiles of 64, exact softmax via the running-max (online) form.
// ---------------------------------------------------------------------------

constexpr int PQ = 64;   // queries per block (one wave)
constexpr int PK = 64;   // keys per tile
constexpr int HDM = 64;  // max head_dim

__global__ __launch_bounds__(64) void attn_prefill_kernel(const float* __restrict__ qkv, int T, int past,
                                                          const float* __restrict__ kc, const float* __restrict__ vc,
                                                          int H, int P, int d, int hd, float* __restrict__ out) {
  __shared__ float Ks[PK][HDM + 1];
  __shared__ float Vs[PK][HDM + 1];
  __shared__ float Ss[PQ][PK + 1];
  const int qb = blockIdx.x, h = blockIdx.y, sidx = blockIdx.z, tid = threadIdx.x;
  const int i = qb * PQ + tid;
  const bool active = i < T;
  const int pabs = past + i;
  const size_t head_off = ((size_t)sidx * H + h) * P * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  float q[HDM], o[HDM];
#pragma unroll
  for (int dd = 0; dd < HDM; ++dd) {
    q[dd] = (active && dd < hd) ? qkv[((size_t)sidx * T + i) * 3 * d + h * hd + dd] : 0.f;
    o[dd] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int last_q = min(T, (qb + 1) * PQ) - 1;
  const int kend = past + last_q;  // inclusive
  for (int j0 = 0; j0 <= kend; j0 += PK) {
    __syncthreads();
    // Stage keys/values j0 .. j0+PK-1 (thread tid loads row j0+tid).
    {
      const int j = j0 + tid;
      for (int dd = 0; dd < HDM; ++dd) {
        const bool ok = j <= kend && dd < hd;
        Ks[tid][dd] = ok ? kc[head_off + (size_t)j * hd + dd] : 0.f;
        Vs[tid][dd] = ok ? vc[head_off + (size_t)j * hd + dd] : 0.f;
      }
    }
    __syncthreads();
    float tmax = -INFINITY;
    for (int jj = 0; jj < PK; ++jj) {
      const int j = j0 + jj;
      float sv = -INFINITY;
      if (active && j <= pabs) {
        float dot = 0.f;
#pragma unroll
        for (int dd = 0; dd < HDM; ++dd) dot = fmaf(q[dd], Ks[jj][dd], dot);
        sv = dot * scale;
      }
      Ss[tid][jj] = sv;
      tmax = fmaxf(tmax, sv);
    }
    if (active && tmax > -INFINITY) {
      const float mn = fmaxf(m, tmax);
      const float corr = expf(m - mn);
      l *= corr;
#pragma unroll
      for (int dd = 0; dd < HDM; ++dd) o[dd] *= corr;
      for (int jj = 0; jj < PK; ++jj) {
        const float sv = Ss[tid][jj];
        if (sv == -INFINITY) continue;
        const float p = expf(sv - mn);
        l += p;
#pragma unroll
        for (int dd = 0; dd < HDM; ++dd) o[dd] = fmaf(p, Vs[jj][dd], o[dd]);
      }
      m = mn;
    }
  }
  if (active) {
    const float inv = 1.0f / l;
    for (int dd = 0; dd < hd; ++dd) out[((size_t)sidx * T + i) * d + h * hd + dd] = o[dd] * inv;
  }
}

// ---------------------------------------------------------------------------
// Prefill causal attention for head_dim 64 on fp32 MFMA (flash-attention
// form of multi_head_attention_cached, gpt2.rs:772-834). A workgroup of FW
// waves takes 32 * FW queries of one (sequence, head); each wave owns 32. Key
// blocks of 32 rows are staged in LDS (K row-major, V transposed), the next
// block's rows are loaded into registers while the current one is used.
//
// Per key block a wave computes S^T = K Q^T (32 keys x 32 queries, 32
// v_mfma_f32_32x32x2f32 steps over the 64 dims: step kk pairs dims kk and
// kk + 32), so accumulator i of lane l holds the score of query l % 32 with
// key r(i, l) = (i/4)*8 + (l/32)*4 + i%4. The softmax statistics of a query
// are therefore lane-local (16 values) plus one exchange between the two
// lane halves, and the rescale of the output is lane-local.
// O^T += V^T P^T runs 16 steps per 32-dim output tile; step kk takes key
// r(kk, l) in lane half l/32, which is exactly accumulator kk of the lane,
// so P feeds the MFMA from registers. Online softmax with running max m and
// per-half partial sums l (combined at the end), as the scalar kernel.
// ---------------------------------------------------------------------------

constexpr int FA_QW = 32;         // queries per wave
constexpr int FA_K = 32;          // keys per block
constexpr int FA_KP = 64 + 4;     // padded K row (floats)
constexpr int FA_VP = FA_K + 4;   // padded V^T row (floats)

template <int FW>
__global__ __launch_bounds__(64 * FW) void attn_prefill_mfma_kernel(
    const float* __restrict__ qkv, int T, int past, const float* __restrict__ kc, const float* __restrict__ vc,
    int H, int P, int d, int nqb, float* __restrict__ out) {
  constexpr int NT = 64 * FW, U = 512 / NT;  // threads; float4 of K (and of V) a thread stages per block
  __shared__ __attribute__((aligned(16))) float Ks[FA_K][FA_KP];
  __shared__ __attribute__((aligned(16))) float Vt[64][FA_VP];
  // the query block is the slowest grid dimension, longest (last) blocks
  // first: every (sequence, head)'s longest block is dispatched before any
  // shorter one, which keeps the tail of the grid short
  const int qb = nqb - 1 - (int)blockIdx.z;
  const int h = blockIdx.x, sidx = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane & 31, hh = lane >> 5;
  const int qi = qb * FA_QW * FW + wave * FA_QW + c;  // this lane's query (0..T-1 when valid)
  const bool qvalid = qi < T;
  const int qpos = past + qi;
  const size_t head_off = ((size_t)sidx * H + h) * (size_t)P * 64;
  const float* Kh = kc + head_off;
  const float* Vh = vc + head_off;
  // this lane's half of its query row: dims [32*hh, 32*hh + 32)
  float q[32];
  {
    const float* qrow = qkv + ((size_t)sidx * T + min(qi, T - 1)) * 3 * d + h * 64 + 32 * hh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 v = reinterpret_cast<const float4*>(qrow)[j];
      q[4 * j] = v.x;
      q[4 * j + 1] = v.y;
      q[4 * j + 2] = v.z;
      q[4 * j + 3] = v.w;
    }
  }
  const int kmax = past + min(T, (qb + 1) * FA_QW * FW) - 1;  // last key any query here attends
  const int nkb = kmax / FA_K + 1;
  // staging: 512 float4 of K and of V per block, U each per thread
  float4 kr[U], vr[U];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + u * NT;
      const int r = e >> 4, c4 = (e & 15) * 4, j = kb * FA_K + r;
      const bool ok = j <= kmax;
      kr[u] = ok ? *reinterpret_cast<const float4*>(Kh + (size_t)j * 64 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
      vr[u] = ok ? *reinterpret_cast<const float4*>(Vh + (size_t)j * 64 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  float m = -INFINITY, l = 0.f;
  floatx16 o0, o1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o0[i] = 0.f;
    o1[i] = 0.f;
  }
  load_block(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();  // every wave is done with the previous block
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + u * NT;
      const int r = e >> 4, c4 = (e & 15) * 4;
      *reinterpret_cast<float4*>(&Ks[r][c4]) = kr[u];
      Vt[c4][r] = vr[u].x;
      Vt[c4 + 1][r] = vr[u].y;
      Vt[c4 + 2][r] = vr[u].z;
      Vt[c4 + 3][r] = vr[u].w;
    }
    __syncthreads();
    if (kb + 1 < nkb) load_block(kb + 1);
    // S^T = K Q^T
    floatx16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 a = *reinterpret_cast<const float4*>(&Ks[c][32 * hh + 4 * j]);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, q[4 * j], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, q[4 * j + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, q[4 * j + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, q[4 * j + 3], s, 0, 0, 0);
    }
    // causal mask (key j <= query position), scale 1/sqrt(64), online softmax
    const int j0 = kb * FA_K;
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = j0 + (i / 4) * 8 + hh * 4 + (i % 4);
      s[i] = j <= qpos ? s[i] * 0.125f : -INFINITY;
      bm = fmaxf(bm, s[i]);
    }
    bm = xor32_max_k(bm);
    const float mn = fmaxf(m, bm);
    const float corr = m == -INFINITY ? 0.f : fexp_a(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = s[i] == -INFINITY ? 0.f : fexp_a(s[i] - mn);
      ps += s[i];
    }
    l = l * corr + ps;
    m = mn;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] *= corr;
      o1[i] *= corr;
    }
    // O^T += V^T P^T
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 v0 = *reinterpret_cast<const float4*>(&Vt[c][8 * g + 4 * hh]);
      const float4 v1 = *reinterpret_cast<const float4*>(&Vt[32 + c][8 * g + 4 * hh]);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.x, s[4 * g], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.x, s[4 * g], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.y, s[4 * g + 1], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.y, s[4 * g + 1], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.z, s[4 * g + 2], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.z, s[4 * g + 2], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.w, s[4 * g + 3], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.w, s[4 * g + 3], o1, 0, 0, 0);
    }
  }
  l = xor32_sum_k(l);
  if (qvalid) {
    const float inv = 1.0f / l;
    float* orow = out + ((size_t)sidx * T + qi) * d + h * 64;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = (i / 4) * 8 + hh * 4 + (i % 4);
      orow[r] = o0[i] * inv;
      orow[32 + r] = o1[i] * inv;
    }
  }
}

// attn_prefill_mfma_kernel with the key range split over the waves: a
// workgroup of KS waves takes 32 queries of one (sequence, head) and wave w
// the key blocks w, w + KS, ... (each staged in the wave's own LDS region, so
// no workgroup barrier per block); the waves' (m, l, O) merge in LDS at the
// end (out = sum_w O_w e^(m_w - M) / sum_w l_w e^(m_w - M)). For a few long
// prompts the causal chain of the last query block (T / 32 key blocks, one
// after the other on one wave) is otherwise the whole kernel.
template <int KS>
__global__ __launch_bounds__(64 * KS) void attn_prefill_ks_kernel(const float* __restrict__ qkv, int T, int past,
                                                                  const float* __restrict__ kc,
                                                                  const float* __restrict__ vc, int H, int P, int d,
                                                                  int nqb, float* __restrict__ out) {
  constexpr int REG = FA_K * FA_KP + 64 * FA_VP;  // floats of one wave's K block and V^T block
  constexpr int MW = 64 + 2;                      // merge record of one query: m, l, O[64]
  static_assert(FA_QW * MW <= REG, "merge records fit the staging region");
  __shared__ __attribute__((aligned(16))) float sm[KS][REG];
  const int qb = nqb - 1 - (int)blockIdx.z;  // longest query blocks first
  const int h = blockIdx.x, sidx = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 31, hh = lane >> 5;
  const int qi = qb * FA_QW + c;
  const bool qvalid = qi < T;
  const int qpos = past + qi;
  const size_t head_off = ((size_t)sidx * H + h) * (size_t)P * 64;
  const float* Kh = kc + head_off;
  const float* Vh = vc + head_off;
  float(*Ks)[FA_KP] = reinterpret_cast<float(*)[FA_KP]>(&sm[wave][0]);
  float(*Vt)[FA_VP] = reinterpret_cast<float(*)[FA_VP]>(&sm[wave][FA_K * FA_KP]);
  float q[32];
  {
    const float* qrow = qkv + ((size_t)sidx * T + min(qi, T - 1)) * 3 * d + h * 64 + 32 * hh;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 v = reinterpret_cast<const float4*>(qrow)[j];
      q[4 * j] = v.x;
      q[4 * j + 1] = v.y;
      q[4 * j + 2] = v.z;
      q[4 * j + 3] = v.w;
    }
  }
  const int kmax = past + min(T, (qb + 1) * FA_QW) - 1;
  const int nkb = kmax / FA_K + 1;
  float4 kr[8], vr[8];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = lane + u * 64;
      const int r = e >> 4, c4 = (e & 15) * 4, j = kb * FA_K + r;
      const bool ok = j <= kmax;
      kr[u] = ok ? *reinterpret_cast<const float4*>(Kh + (size_t)j * 64 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
      vr[u] = ok ? *reinterpret_cast<const float4*>(Vh + (size_t)j * 64 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  float m = -INFINITY, l = 0.f;
  floatx16 o0, o1;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    o0[i] = 0.f;
    o1[i] = 0.f;
  }
  if (wave < nkb) load_block(wave);
  for (int kb = wave; kb < nkb; kb += KS) {
    // this wave's region only: LDS accesses of one wave are ordered, the
    // wave's previous reads are complete before its writes below
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = lane + u * 64;
      const int r = e >> 4, c4 = (e & 15) * 4;
      *reinterpret_cast<float4*>(&Ks[r][c4]) = kr[u];
      Vt[c4][r] = vr[u].x;
      Vt[c4 + 1][r] = vr[u].y;
      Vt[c4 + 2][r] = vr[u].z;
      Vt[c4 + 3][r] = vr[u].w;
    }
    if (kb + KS < nkb) load_block(kb + KS);
    floatx16 sc;
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 a = *reinterpret_cast<const float4*>(&Ks[c][32 * hh + 4 * j]);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, q[4 * j], sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, q[4 * j + 1], sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, q[4 * j + 2], sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, q[4 * j + 3], sc, 0, 0, 0);
    }
    const int j0 = kb * FA_K;
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int j = j0 + (i / 4) * 8 + hh * 4 + (i % 4);
      sc[i] = j <= qpos ? sc[i] * 0.125f : -INFINITY;
      bm = fmaxf(bm, sc[i]);
    }
    bm = xor32_max_k(bm);
    const float mn = fmaxf(m, bm);
    const float corr = m == -INFINITY ? 0.f : fexp_a(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sc[i] = sc[i] == -INFINITY ? 0.f : fexp_a(sc[i] - mn);
      ps += sc[i];
    }
    l = l * corr + ps;
    m = mn;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] *= corr;
      o1[i] *= corr;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 v0 = *reinterpret_cast<const float4*>(&Vt[c][8 * g + 4 * hh]);
      const float4 v1 = *reinterpret_cast<const float4*>(&Vt[32 + c][8 * g + 4 * hh]);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.x, sc[4 * g], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.x, sc[4 * g], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.y, sc[4 * g + 1], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.y, sc[4 * g + 1], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.z, sc[4 * g + 2], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.z, sc[4 * g + 2], o1, 0, 0, 0);
      o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(v0.w, sc[4 * g + 3], o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(v1.w, sc[4 * g + 3], o1, 0, 0, 0);
    }
  }
  l = xor32_sum_k(l);
  // merge records: query c of wave w at sm[w][c * MW]: m, l, O[64]
  __syncthreads();  // every wave is done with its staging region
  float* rec = &sm[wave][c * MW];
  if (hh == 0) {
    rec[0] = m;
    rec[1] = l;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = (i / 4) * 8 + hh * 4 + (i % 4);
    rec[2 + r] = o0[i];
    rec[2 + 32 + r] = o1[i];
  }
  __syncthreads();
  // wave 0 lane (c, hh) merges the 32 dims it holds for query c
  if (wave == 0 && qvalid) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < KS; ++w) M = fmaxf(M, sm[w][c * MW]);
    float L = 0.f, f[KS];
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      const float mw = sm[w][c * MW];
      f[w] = mw == -INFINITY ? 0.f : fexp_a(mw - M);
      L += sm[w][c * MW + 1] * f[w];
    }
    const float inv = 1.0f / L;
    float* orow = out + ((size_t)sidx * T + qi) * d + h * 64;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = (i / 4) * 8 + hh * 4 + (i % 4);
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int w = 0; w < KS; ++w) {
        a += sm[w][c * MW + 2 + r] * f[w];
        b += sm[w][c * MW + 2 + 32 + r] * f[w];
      }
      orow[r] = a * inv;
      orow[32 + r] = b * inv;
    }
  }
}

void launch_attn_prefill(hipStream_t s, const float* qkv, int S, int T, int past, const float* kc, const float* vc,
                         int n_head, int n_pos, int d, float* out) {
  if (d / n_head == 64 && (long)n_head * S < 256 && T + past >= 4 * FA_K) {
    // few (sequence, head) pairs with long key ranges: split the keys over 4
    // waves, 8 from 16 key blocks on (c3, 512 tokens of GPT-2 medium: 85.4k
    // -> 96.9k tokens/s with 4, 5.25 -> 5.10-5.23 ms with 8; c2, 8 x 128
    // tokens: 3.885 -> 3.82 ms with 4)
    const int nqb = (T + FA_QW - 1) / FA_QW;
    const dim3 grid(n_head, S, nqb);
    if (T + past >= 16 * FA_K)
      attn_prefill_ks_kernel<8><<<grid, 512, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, nqb, out);
    else
      attn_prefill_ks_kernel<4><<<grid, 256, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, nqb, out);
    return;
  }
  if (d / n_head == 64) {
    // 128 queries per workgroup where that gives two workgroups per CU, else
    // 64 or 32 (a short batch of prompts would otherwise leave most CUs idle)
    int fw = 4;
    while (fw > 1 && (long)n_head * S * ((T + FA_QW * fw - 1) / (FA_QW * fw)) < 512) fw >>= 1;
    const int nqb = (T + FA_QW * fw - 1) / (FA_QW * fw);
    dim3 grid(n_head, S, nqb);
    if (fw == 4)
      attn_prefill_mfma_kernel<4><<<grid, 256, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, nqb, out);
    else if (fw == 2)
      attn_prefill_mfma_kernel<2><<<grid, 128, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, nqb, out);
    else
      attn_prefill_mfma_kernel<1><<<grid, 64, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, nqb, out);
    return;
  }
  dim3 grid((T + PQ - 1) / PQ, n_head, S);
  attn_prefill_kernel<<<grid, PQ, 0, s>>>(qkv, T, past, kc, vc, n_head, n_pos, d, d / n_head, out);
}

// ---------------------------------------------------------------------------
// Load-time layout conversion: [rows][cols] -> [cols][rows] (Conv1D [in][out]
// -> W^T [out][in]) and plain conversion, from the file's element type (f32,
// bf16 or f16, so that bf16 / f16 weights are uploaded as they are stored and
// widened here) to the storage type (f32, or bf16 rounded to nearest even).
// bf16 -> f32 is bf16_to_f32 (bits << 16, nn/safetensors.rs:389-391); f16 ->
// f32 is the exact IEEE conversion.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

__device__ __forceinline__ float load_elem(const void* src, int stype, size_t i) {
  if (stype == SRC_F32) return static_cast<const float*>(src)[i];
  const uint16_t h = static_cast<const uint16_t*>(src)[i];
  if (stype == SRC_BF16) return __uint_as_float((uint32_t)h << 16);
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}

__device__ __forceinline__ void store_elem(void* dst, int wtype, size_t i, float v) {
  if (wtype == W_F32) static_cast<float*>(dst)[i] = v;
  else static_cast<uint16_t*>(dst)[i] = f32_to_bf16_rne(v);
}

__global__ void transpose_kernel(const void* __restrict__ src, int stype, int rows, int cols, void* __restrict__ dst,
                                 int wtype) {
  __shared__ float tile[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int y = ty; y < 32; y += 8) {
    const int r = r0 + y, c = c0 + tx;
    tile[y][tx] = (r < rows && c < cols) ? load_elem(src, stype, (size_t)r * cols + c) : 0.f;
  }
  __syncthreads();
  for (int y = ty; y < 32; y += 8) {
    const int c = c0 + y, r = r0 + tx;  // dst[c][r]
    if (c < cols && r < rows) store_elem(dst, wtype, (size_t)c * rows + r, tile[tx][y]);
  }
}

void launch_transpose_to(hipStream_t s, const void* src, int stype, int rows, int cols, void* dst, int wtype) {
  dim3 grid((cols + 31) / 32, (rows + 31) / 32);
  transpose_kernel<<<grid, 256, 0, s>>>(src, stype, rows, cols, dst, wtype);
}

__global__ void convert_kernel(const void* __restrict__ src, int stype, long n, void* __restrict__ dst, int wtype) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    store_elem(dst, wtype, (size_t)i, load_elem(src, stype, (size_t)i));
}

void launch_convert_to(hipStream_t s, const void* src, int stype, long n, void* dst, int wtype) {
  long blocks = (n + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  if (blocks < 1) blocks = 1;
  convert_kernel<<<(unsigned)blocks, 256, 0, s>>>(src, stype, n, dst, wtype);
}

}  // namespace rtg
