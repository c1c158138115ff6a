// Batched decode GEMV (2..16 sequences) over tile-ordered weights; see
// bgemv.hip for the tile layout and the work split.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace rtg {

// QKV epilogue target: q part to q[m][ldq], the new token's k/v parts into
// the cache at *pos_dev. q == nullptr selects the plain epilogues.
struct BgemvQkv {
  float* q;
  int ldq;
  int d;
  KvDst kv;
  const int* pos_dev;
};

struct BgemvArgs {
  // f32 inputs of M <= 16 rows in the GEMV input layout: element (m, k) at
  // xt_index(m, k, M, TK) (kernels.h), TK = 16 for f32 weights, 32 for bf16
  const float* X;
  int M;
  const void* Wt;  // tile-ordered weights (launch_tile_weights)
  int wtype, N, K;
  const float* bias;  // [N] or null
  float* C;           // [M][ldc] output (plain epilogues)
  long ldc;
  int epi;
  // C written in the input layout of the next GEMV instead (xt_index with
  // this GEMV's M and TK; ldc unused): the gelu_new epilogue of c_fc, whose
  // output only the MLP projection reads. Not with the residual or QKV
  // epilogues.
  bool c_tiled;
  BgemvQkv qkv;
  // LayerNorm folded in (ln_g set): X holds x already scaled by the gain
  // ln_g[k] (written so by the kernel that produced x, see xg below), and the
  // epilogue computes inv_std * (acc - mean * ln_s[n]) before the bias (then
  // the folded constant c[n]). The statistics of input row m come from the
  // partials the kernel that wrote x left in ln_part[g][m] = (mean, M2) over
  // columns [g * ln_cols, (g + 1) * ln_cols) of K, g < ln_groups <= 128.
  const float* ln_g;
  const float* ln_s;
  const float* ln_part;
  int ln_groups, ln_cols;
  float eps;
  // Centring of the folded LayerNorm: X holds (x - cen_in[m]) * g (the
  // producer subtracted that centre), so the epilogue computes
  // inv_std * (acc - (mean - cen_in[m]) * ln_s[n]) and no term carries the
  // row's full mean (null: centre 0). cen_out[m] receives the row's exact
  // mean (written once, by the workgroup of panel group 0): the centre of
  // the next residual producer.
  const float* cen_in;
  float* cen_out;
  // Residual epilogue only: writes those partials for the rows it wrote,
  // stats_part[g][m] for its panel groups g (plan.groups * 32 floats), with
  // groups of 16 * plan.npw columns; with xg set, also y * g_next[n] to xg in
  // the input layout (xt_index(m, n, M, TK)), the input of the next
  // LayerNorm-folded GEMV.
  float* stats_part;
  float* xg;
  const float* g_next;
  // with xg: (y - xg_cen[m]) * g_next[n] is written instead (null: centre 0)
  const float* xg_cen;
  // LM head: per-row packed argmax keys (gpt2.rs:858-868), updated with a
  // device-scope atomic max (zero before; the step's finalize resets them).
  unsigned long long* keys;
  float* part;    // workspace of bgemv_work_floats(plan) floats when plan.S > 1
  unsigned* cnt;  // plan.groups zeroed counters when plan.S > 1 (left zeroed)
  int S, ktc;     // filled in from the plan
};

struct BgemvPlan {
  int npw;     // 16-row panels per wave
  int S;       // workgroups per panel group (k splits)
  int ktc;     // k-tiles per wave
  int groups;  // panel groups
};

// Bytes of the tile-ordered copy of W^T[N][K] (rows padded to 16).
size_t tiled_weight_bytes(int N, int K, int wtype);
// Writes the tile-ordered copy of a row-major W^T[N][K] in storage type wtype.
bool launch_tile_weights(hipStream_t s, const void* src, int wtype, int N, int K, void* dst);
// Work split for one GEMV shape with nw waves per workgroup; npw_force /
// s_force > 0 override the choice.
BgemvPlan bgemv_plan(int N, int K, int wtype, int npw_force = 0, int s_force = 0, int nw = 4);
// The argument checks launch_bgemv makes (shape, workspaces, LayerNorm parts).
bool bgemv_args_ok(const BgemvPlan& pl, const BgemvArgs& a);
size_t bgemv_work_floats(const BgemvPlan& pl);
bool launch_bgemv(hipStream_t s, const BgemvPlan& pl, BgemvArgs a);
// Decode embedding x[r] = wte[token[r]] + wpe[*pos_dev] of rows r < rows,
// (x[r] - mean_r) * g in the GEMV input layout to xg (xt_index(r, k, rows,
// TK of wtype): the input of the LayerNorm-folded GEMV that follows, centred
// on the row's mean, cen[r] = mean_r) and their LayerNorm statistics
// partials as one group of width d: part[r] = (mean, M2) (the ln_part of the
// following GEMV, ln_groups = 1). d <= 2048.
bool launch_embed_stats(hipStream_t s, const void* wte, int wtype, const float* wpe, const uint32_t* token,
                        const int* pos_dev, int rows, int d, float* x, float* part, const float* g,
                        float* xg, float* cen);

}  // namespace rtg
