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
// f32 tiles: MFMA step e of a tile pairs k = t*TK + q*E + e for q = 0..3, so
// lane l's A operand is x[r][t*TK + q*E + e] and it accumulates D[4q + i][r],
// i < 4 (batch row 4q + i, output row 16p + r). bf16 tiles: the lane's 16
// bytes are the B operand of one v_mfma_f32_16x16x32_bf16 (k = t*TK + 8q +
// 0..7); x[r][those k] enters as three exact bf16 parts (hi, mid, lo: three
// MFMAs per tile, all products exact), the same D layout.
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
#include "bgemv_core.h"

namespace rtg {

namespace {

using bgc::u4v;
constexpr int BG_NW = 4;  // waves per workgroup of the standalone kernel

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

template <int WT, int NPW, bool LNG, int DEPTH, bool ONESHOT>
__global__ __launch_bounds__(64 * BG_NW) void bgemv_kernel(BgemvArgs a) {
  __shared__ float red[BG_NW][NPW][256];
  __shared__ unsigned last;
  bgc::bgemv_unit<WT, NPW, LNG, BG_NW, DEPTH, ONESHOT>(a, blockIdx.x, blockIdx.y, red, &last);
}

// k-tiles a wave keeps in flight: its whole chunk at once when that fits
// the register budget (about 160 registers of tiles: weights and x), else a
// ring of 4.
int bgemv_depth(const BgemvPlan& pl, int wtype) {
  const int per_tile = 4 * pl.npw + (wtype == W_F32 ? 4 : 8);
  for (int d : {8, 12})
    if (pl.ktc <= d && per_tile * d <= 160) return d;
  return 4;
}

// Decode embedding of B rows (gpt2.rs:377-384: wte[token] + wpe[position]),
// x * g in the GEMV input layout, and the rows' LayerNorm statistics
// partials as one group of width d
// (part[m] = (mean, M2), two passes as layer_norm, gpt2.rs:636-666): one
// workgroup of 256 threads per row.
__global__ __launch_bounds__(256) void embed_stats_kernel(const void* __restrict__ wte, int wtype,
                                                          const float* __restrict__ wpe,
                                                          const uint32_t* __restrict__ token,
                                                          const int* __restrict__ pos_dev, int d,
                                                          float* __restrict__ x, float* __restrict__ part,
                                                          const float* __restrict__ g, float* __restrict__ xg,
                                                          float* __restrict__ cen) {
  __shared__ float red[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int tk = wtype == W_F32 ? 16 : 32;  // xg in the GEMV input layout
  const long tok = token[b];
  const int pos = *pos_dev;
  float v[8];  // d <= 2048
  float s = 0.f;
  // every load of the row in flight at once (branch-free: lanes past the
  // row's end re-read its last element and drop it), then the stores
  float w[8], pe[8], gk[8];
  if (wtype == W_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = static_cast<const float*>(wte)[tok * d + min(tid + 256 * i, d - 1)];
  } else {
    uint32_t wb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) wb[i] = static_cast<const uint16_t*>(wte)[tok * d + min(tid + 256 * i, d - 1)];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __uint_as_float(wb[i] << 16);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = min(tid + 256 * i, d - 1);
    pe[i] = wpe[(long)pos * d + k];
    gk[i] = g[k];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = tid + 256 * i;
    v[i] = 0.f;
    if (k < d) {
      v[i] = w[i] + pe[i];
      x[(long)b * d + k] = v[i];
      s += v[i];
    }
  }
  auto block_sum = [&](float t) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = t;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
  };
  const float mean = block_sum(s) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = v[i] - mean;
    q += tid + 256 * i < d ? t * t : 0.f;
  }
  q = block_sum(q);
  // the GEMV input centred on the row's own mean: (x - mean) * g, so that the
  // folded LayerNorm of the next GEMV subtracts no large mean (cen[b] = the
  // centre used)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = tid + 256 * i;
    if (k < d) xg[xt_index(b, k, gridDim.x, tk)] = (v[i] - mean) * gk[i];
  }
  if (tid == 0) {
    part[2 * b] = mean;
    part[2 * b + 1] = q;
    cen[b] = mean;
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

BgemvPlan bgemv_plan(int N, int K, int wtype, int npw_force, int s_force, int nw) {
  // Measured on MI355X over the GPT-2 decode shapes (2304..50257 rows, K 768..6400,
  // f32 and bf16, whole decode steps): two panels per wave once there are >= 300
  // panels (for the LM head four with bf16 weights, one with f32: 29.6 against
  // 33.3 µs with two), one below; K >= 150 tiles (the MLP projection) splits
  // the k range over 5 workgroups with two panels per wave for bf16 (c5 2138 ->
  // 2104 µs per step against one panel; 4 splits 2215) and over 4 for f32 (c2
  // 380 -> 377 µs against 5); shorter k ranges are not split (the attention
  // projection: c2 390 -> 380 µs against 2 splits).
  BgemvPlan pl{};
  const int TK = wtype == W_F32 ? 16 : 32;
  const int KT = K / TK, NP = (N + 15) / 16;
  const bool bf = wtype == W_BF16;
  pl.npw = npw_force > 0 ? npw_force : (NP >= 1500 ? (bf ? 4 : 1) : NP >= 300 || (bf && KT >= 150) ? 2 : 1);
  int S = s_force > 0 ? s_force : (KT >= 150 ? (bf ? 5 : 4) : 1);
  if (S < 1) S = 1;
  if (S > bgc::SMAX) S = bgc::SMAX;
  pl.ktc = (KT + S * nw - 1) / (S * nw);
  // every workgroup must own at least one tile so that all S arrive
  while (S > 1 && (S - 1) * nw * pl.ktc >= KT) {
    --S;
    pl.ktc = (KT + S * nw - 1) / (S * nw);
  }
  pl.S = S;
  pl.groups = (NP + pl.npw - 1) / pl.npw;
  return pl;
}

bool bgemv_args_ok(const BgemvPlan& pl, const BgemvArgs& a) {
  const int TK = a.wtype == W_F32 ? 16 : 32;
  if (a.M < 1 || a.M > 16 || a.K % TK != 0) return false;
  if (a.c_tiled && (a.epi == EPI_BIAS_RESID || a.qkv.q || a.N % TK != 0)) return false;
  if (pl.S < 1 || pl.S > bgc::SMAX || (pl.S > 1 && (!a.part || !a.cnt))) return false;
  if (a.ln_g && (!a.ln_s || !a.ln_part || a.ln_groups < 1 || a.ln_groups > 16 * bgc::LNG_PER || a.ln_cols < 1 ||
                 (a.ln_groups - 1) * a.ln_cols >= a.K || a.ln_groups * a.ln_cols < a.K))
    return false;
  if (a.stats_part && a.epi != EPI_BIAS_RESID) return false;
  if ((a.cen_in || a.cen_out) && !a.ln_g) return false;
  if (a.xg_cen && !a.xg) return false;
  return true;
}

size_t bgemv_work_floats(const BgemvPlan& pl) { return pl.S > 1 ? (size_t)pl.groups * pl.S * pl.npw * 256 : 0; }

bool launch_bgemv(hipStream_t s, const BgemvPlan& pl, BgemvArgs a) {
  if (!bgemv_args_ok(pl, a)) return false;
  a.S = pl.S;
  a.ktc = pl.ktc;
  const dim3 grid(pl.groups, pl.S);
  const dim3 block(64 * BG_NW);
  const int depth = bgemv_depth(pl, a.wtype);
#define BG_LAUNCH_D(WT, NPW, LNG)                                                         \
  do {                                                                                    \
    if (depth == 12) bgemv_kernel<WT, NPW, LNG, 12, true><<<grid, block, 0, s>>>(a);      \
    else if (depth == 8) bgemv_kernel<WT, NPW, LNG, 8, true><<<grid, block, 0, s>>>(a);   \
    else bgemv_kernel<WT, NPW, LNG, 4, false><<<grid, block, 0, s>>>(a);                  \
  } while (0)
#define BG_LAUNCH(WT, NPW)                 \
  do {                                     \
    if (a.ln_g) BG_LAUNCH_D(WT, NPW, true); \
    else BG_LAUNCH_D(WT, NPW, false);       \
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
#undef BG_LAUNCH_D
  return hipGetLastError() == hipSuccess;
}

bool launch_embed_stats(hipStream_t s, const void* wte, int wtype, const float* wpe, const uint32_t* token,
                        const int* pos_dev, int rows, int d, float* x, float* part, const float* g,
                        float* xg, float* cen) {
  if (d > 2048 || d % (wtype == W_F32 ? 16 : 32) != 0) return false;
  embed_stats_kernel<<<rows, 256, 0, s>>>(wte, wtype, wpe, token, pos_dev, d, x, part, g, xg, cen);
  return hipGetLastError() == hipSuccess;
}

}  // namespace rtg
