// Host side of the tiled persistent decode step (decode_tile_kernel.h): the
// per-workgroup weight tiles, the block-folded LayerNorm constants, the
// tagged exchange layout, and the kernel instance.
//
// Tile layouts (f4v = 4 floats of one W^T row; t = task = GEMV lane of the
// workgroup, i = float4 index within the task; each tile is [i][t] so that
// a wave's i-th load reads 64 consecutive float4 = 1 KiB):
//   c_attn  tile (h, c), h < H: task t = head-major row (q rows 0..63, k rows
//           64..127, v rows 128..191 of head h), columns [CB c + 4i, +4)
//   attn c_proj tile (h, c): task t = 4 jj + q: row CB c + jj, columns
//           [64 h + 16 q + 4 i, +4) (i < 4)
//   c_fc    tile (r, c): task t: row HB r + t, columns [CB c + 4i, +4)
//   mlp c_proj tile (r, c): task t = 4 jj + q: row CB r + jj, columns
//           [HB c + CB q + 4 i, +4)
// Tile (r, c) of every matrix lives at offset (16 r + c) * NV * NT (float4).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "decode_tile.h"
#include "decode_tile_kernel.h"

namespace rtg {

namespace {

enum { TM_QKV = 0, TM_PROJ = 1, TM_FC = 2, TM_MLP = 3 };

// Source row (of W^T) and first column of float4 e of the tiles of `mode`.
__device__ __forceinline__ void tile_src(int mode, long e, int D, int& row, int& col) {
  const int CB = D / tk::GS, HB = 4 * D / tk::GS, NV = CB / 4;
  if (mode == TM_QKV) {
    const int NT = 3 * tk::HD;
    const int t = (int)(e % NT);
    const long wi = e / NT;
    const int i = (int)(wi % NV), w = (int)(wi / NV);
    const int h = w >> 4, c = w & 15;
    row = (t / tk::HD) * D + tk::HD * h + t % tk::HD;
    col = CB * c + 4 * i;
  } else if (mode == TM_PROJ) {
    const int NT = 4 * CB, NVP = tk::HD / 16;
    const int t = (int)(e % NT);
    const long wi = e / NT;
    const int i = (int)(wi % NVP), w = (int)(wi / NVP);
    const int h = w >> 4, c = w & 15;
    row = CB * c + (t >> 2);
    col = tk::HD * h + 16 * (t & 3) + 4 * i;
  } else if (mode == TM_FC) {
    const int NT = HB;
    const int t = (int)(e % NT);
    const long wi = e / NT;
    const int i = (int)(wi % NV), w = (int)(wi / NV);
    row = HB * (w >> 4) + t;
    col = CB * (w & 15) + 4 * i;
  } else {
    const int NT = 4 * CB;
    const int t = (int)(e % NT);
    const long wi = e / NT;
    const int i = (int)(wi % NV), w = (int)(wi / NV);
    row = CB * (w >> 4) + (t >> 2);
    col = HB * (w & 15) + CB * (t & 3) + 4 * i;
  }
}

__global__ void tile_gather_kernel(const float* W, int K, int mode, int D, float4* dst, long n4) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n4) return;
  int row, col;
  tile_src(mode, e, D, row, col);
  dst[e] = *reinterpret_cast<const float4*>(W + (long)row * K + col);
}

// Block-folded LayerNorm constants of W^T [N][K] (K = D): for output row j
// (head-major for c_attn), s[j][c] = sum_{k in block c} W[n][k] g[k] and
// c[j] = bias[n] + sum_k W[n][k] b[k], accumulated in double. One thread per
// (row, block) pair; block GS is the constant.
__global__ void tile_fold_kernel(const float* W, int N, int D, int headmajor, const float* g, const float* b,
                                 const float* bias, float* s, float* cst) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (long)N * (tk::GS + 1)) return;
  const int j = (int)(e / (tk::GS + 1)), c = (int)(e % (tk::GS + 1));
  int n = j;
  if (headmajor) {
    const int QR = 3 * tk::HD;
    const int h = j / QR, r = j % QR;
    n = (r / tk::HD) * D + tk::HD * h + r % tk::HD;
  }
  const float* wr = W + (long)n * D;
  if (c < tk::GS) {
    const int CB = D / tk::GS;
    double acc = 0.0;
    for (int k = CB * c; k < CB * c + CB; ++k) acc += (double)wr[k] * (double)g[k];
    s[(long)j * tk::GS + c] = (float)acc;
  } else {
    double acc = bias ? (double)bias[n] : 0.0;
    for (int k = 0; k < D; ++k) acc += (double)wr[k] * (double)b[k];
    cst[j] = (float)acc;
  }
}

// cl[v] = sum_k wte[v][k] bf[k] (ln_f's bias through the tied LM head), in double.
__global__ void tile_lm_const_kernel(const float* wte, int V, int D, const float* bf, float* cl) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= V) return;
  double acc = 0.0;
  for (int k = 0; k < D; ++k) acc += (double)wte[(long)v * D + k] * (double)bf[k];
  cl[v] = (float)acc;
}

bool gather(const void* W, int K, int mode, int D, float4* dst, long n4) {
  hipLaunchKernelGGL(tile_gather_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, 0,
                     static_cast<const float*>(W), K, mode, D, dst, n4);
  return hipGetLastError() == hipSuccess;
}

}  // namespace

bool tile_supported(int d, int H, int V, int wtype, int cus) {
  return wtype == W_F32 && d == 768 && H * tk::HD == d && V == 50257 && cus >= tk::G;
}

TilePlan* tile_plan_create(const PersistentWeights& w) {
  const int d = (int)w.cfg.n_embd, H = (int)w.cfg.n_head, V = (int)w.cfg.vocab_size, L = (int)w.cfg.n_layer;
  typedef tk::TCfg<768, 50257> C;
  if (d != C::D || V != C::V || H != C::H) return nullptr;
  TilePlan* tp = new TilePlan();
  const long nq = (long)tk::GS * H * C::NV * C::NT_Q, np = (long)tk::GS * H * C::NVP * C::NT_P;
  const long nf = (long)tk::G * C::NV * C::NT_F, nm = (long)tk::G * C::NV * C::NT_M;
  const long per_layer4 = nq + np + nf + nm;  // float4
  const long fold_floats = (long)(3 * d) * (tk::GS + 1) + (long)(4 * d) * (tk::GS + 1);
  const size_t bytes = (size_t)per_layer4 * 16 * L + (size_t)fold_floats * 4 * L + (size_t)V * 4 + 4096;
  if (hipDeviceSynchronize() != hipSuccess || hipMalloc(&tp->arena, bytes) != hipSuccess) {
    tile_plan_destroy(tp);
    return nullptr;
  }
  char* cur = static_cast<char*>(tp->arena);
  std::vector<tk::TLayer> lay(L);
  bool ok = true;
  for (int l = 0; l < L && ok; ++l) {
    const PersistentLayer& s = w.layers[l];
    float4* q = reinterpret_cast<float4*>(cur);
    float4* pp = q + nq;
    float4* f = pp + np;
    float4* m = f + nf;
    cur = reinterpret_cast<char*>(m + nm);
    float* sq = reinterpret_cast<float*>(cur);
    float* cq = sq + (long)(3 * d) * tk::GS;
    float* sf = cq + 3 * d;
    float* cf = sf + (long)(4 * d) * tk::GS;
    cur = reinterpret_cast<char*>(cf + 4 * d);
    ok = gather(s.wqkv, d, TM_QKV, d, q, nq) && gather(s.waproj, d, TM_PROJ, d, pp, np) &&
         gather(s.wfc, d, TM_FC, d, f, nf) && gather(s.wmproj, 4 * d, TM_MLP, d, m, nm);
    const long eq = (long)(3 * d) * (tk::GS + 1), ef = (long)(4 * d) * (tk::GS + 1);
    hipLaunchKernelGGL(tile_fold_kernel, dim3((unsigned)((eq + 255) / 256)), dim3(256), 0, 0,
                       static_cast<const float*>(s.wqkv), 3 * d, d, 1, s.ln1w, s.ln1b, s.bqkv, sq, cq);
    hipLaunchKernelGGL(tile_fold_kernel, dim3((unsigned)((ef + 255) / 256)), dim3(256), 0, 0,
                       static_cast<const float*>(s.wfc), 4 * d, d, 0, s.ln2w, s.ln2b, s.bfc, sf, cf);
    ok = ok && hipGetLastError() == hipSuccess;
    lay[l] = {reinterpret_cast<const pk::f4v*>(q), reinterpret_cast<const pk::f4v*>(pp), reinterpret_cast<const pk::f4v*>(f),
              reinterpret_cast<const pk::f4v*>(m), sq, cq, sf, cf, s.baproj, s.bmproj, s.ln1w, s.ln2w};
  }
  float* cl = reinterpret_cast<float*>(cur);
  hipLaunchKernelGGL(tile_lm_const_kernel, dim3((V + 255) / 256), dim3(256), 0, 0, static_cast<const float*>(w.wte),
                     V, d, w.lnfb, cl);
  ok = ok && hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess;
  if (ok) ok = hipMalloc(&tp->layers_dev, sizeof(tk::TLayer) * L) == hipSuccess;
  if (ok) ok = hipMemcpy(tp->layers_dev, lay.data(), sizeof(tk::TLayer) * L, hipMemcpyHostToDevice) == hipSuccess;
  if (!ok) {
    tile_plan_destroy(tp);
    return nullptr;
  }
  tk::TParams& p = tp->base;
  p.layers = tp->layers_dev;
  p.wte = static_cast<const float*>(w.wte);
  p.wpe = w.wpe;
  p.gf = w.lnfw;
  p.cl = cl;
  p.L = L;
  p.P = (int)w.cfg.n_positions;
  p.eps = w.cfg.layer_norm_epsilon;
  p.kv_layer = (long)H * p.P * tk::HD;
  p.o_q = 0;
  p.o_p = p.o_q + (long)tk::GS * H * C::SQ;
  p.o_f = p.o_p + (long)tk::GS * H * C::SP;
  p.o_m = p.o_f + (long)tk::G * C::SF;
  p.lw = p.o_m + (long)tk::G * C::SM;
  p.o_x = p.lw * L;
  tp->tag_words = (size_t)p.o_x + (size_t)tk::GS * C::SX;
  tp->kernel = (const void*)tk::decode_tile_kernel<768, 50257>;
  return tp;
}

void tile_plan_destroy(TilePlan* tp) {
  if (!tp) return;
  if (tp->layers_dev) hipFree(tp->layers_dev);
  if (tp->arena) hipFree(tp->arena);
  delete tp;
}

int tile_max_len() { return tk::LMAX; }

hipError_t tile_decode_step(const TilePlan* tp, const tk::TParams& p, hipStream_t stream, bool cooperative) {
  void* args[] = {const_cast<tk::TParams*>(&p)};
  if (cooperative)
    return hipLaunchCooperativeKernel(tp->kernel, dim3(tk::G), dim3(tk::NTHREADS), args, 0, stream);
  return hipLaunchKernel(tp->kernel, dim3(tk::G), dim3(tk::NTHREADS), args, 0, stream);
}

}  // namespace rtg
