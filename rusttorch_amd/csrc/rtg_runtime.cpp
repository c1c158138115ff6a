// Host runtime of the GPT-2 token loop on MI355X, exported through the C ABI
// in include/rtgpu.h. It owns HBM-resident weights and KV caches and drives
// the gfx950 kernels of kernels.hip; it never computes model math on the CPU
// (sampling of non-greedy generation aside, which the reference also does on
// the host, gpt2.rs:871-1017).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/rtgpu.h"
#include "decode_persistent.h"
#include "bgemv.h"
#include "kernels.h"
#include "rows.h"
#include "safetensors_reader.h"
#include "scratch.h"

using namespace rtg;

namespace {

rtg_result ok() { return rtg_result{true, nullptr}; }

rtg_result err(const std::string& m) {
  char* s = (char*)malloc(m.size() + 1);
  memcpy(s, m.c_str(), m.size() + 1);
  return rtg_result{false, s};
}

std::string fmt(const char* f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

// A C++ exception other than HipError (e.g. std::bad_alloc for a malformed
// tensor shape) as an error result: no exception crosses the C boundary.
rtg_result err_internal(const std::exception& ex) { return err(std::string("internal error: ") + ex.what()); }

struct HipError {
  std::string msg;
};

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw HipError{std::string("HIP error in ") + what + ": " + hipGetErrorString(e)};
}
#define HIPX(call) hip_check((call), #call)

std::string check_device() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
    return "no HIP device available: rtgpu requires an MI355X (gfx950) GPU";
  int dev = 0;
  hipGetDevice(&dev);
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return "hipGetDeviceProperties failed";
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return std::string("rtgpu is built for gfx950 (MI355X); found ") + prop.gcnArchName;
  return "";
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------

struct LayerW {
  void *wqkv, *waproj, *wfc, *wmproj;  // W^T [N][K] in storage type
  float *bqkv, *baproj, *bfc, *bmproj;
  float *ln1w, *ln1b, *ln2w, *ln2b;
};

// Tile-ordered copies of the decode GEMV weights and the folded LayerNorm
// constants for the batched decode step (bgemv.h), built on first use.
struct BatchedWeights {
  void* arena = nullptr;
  struct Layer {
    const void *qkv, *proj, *fc, *mproj;  // tiled W^T
    const float *sq, *cq, *sf, *cf;       // LN1 into c_attn, LN2 into c_fc
  };
  std::vector<Layer> layers;
  const void* lm = nullptr;  // tiled wte (the tied LM head)
  const float *sl = nullptr, *cl = nullptr;  // ln_f into the LM head
  BgemvPlan pq{}, pp{}, pf{}, pm{}, pl{};    // c_attn, attn c_proj, c_fc, mlp c_proj, LM head
  ~BatchedWeights() {
    if (arena) hipFree(arena);
  }
};

struct rtg_model {
  rtg_config cfg;
  int hd = 0;
  int wtype = W_F32;
  int device = 0;
  void* arena = nullptr;
  size_t arena_bytes = 0;
  void* wte = nullptr;
  float* wpe = nullptr;
  float *lnfw = nullptr, *lnfb = nullptr;
  std::vector<LayerW> layers;
  size_t nparams = 0;
  PersistentPlan* pplan = nullptr;
  RowsPlan* rplan = nullptr;  // multi-row forward (short prompts), null where unsupported
  std::mutex bw_mu;
  std::unique_ptr<BatchedWeights> bw;
  // Pool of caches reused by the generate entry points (keyed by batch).
  std::mutex pool_mu;
  std::multimap<size_t, rtg_cache*> pool;
  ~rtg_model();
};

// ---------------------------------------------------------------------------
// Cache (+ per-cache stream, work buffers and the captured decode graph)
// ---------------------------------------------------------------------------

struct rtg_cache {
  const rtg_model* m = nullptr;
  size_t batch = 1;
  size_t len = 0;
  hipStream_t stream = nullptr;
  float* k = nullptr;  // [L][B][H][P][hd]
  float* v = nullptr;
  size_t layer_stride = 0;  // floats per layer per K (or V)
  // decode state in device memory
  int* pos_dev = nullptr;
  int* step_dev = nullptr;
  unsigned long long* keys = nullptr;
  uint32_t* token_dev = nullptr;
  uint32_t* ids_dev = nullptr;   // [B][P] generated ids
  uint32_t* ids_in = nullptr;    // [B*P] prompt ids
  // work buffers, capacity in rows
  size_t rows_cap = 0;
  float *x = nullptr, *ln = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr;
  float* ws = nullptr;  // split-k partial tiles of the prefill GEMMs
  size_t ws_floats = 0;
  size_t logit_rows_cap = 0;
  float* logits = nullptr;
  // decode graph over the current buffers
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  PersistentState* pstate = nullptr;
  RowsState* rstate = nullptr;  // the multi-row forward's flags and work rows
  // batched decode step (bgemv): split-k partials and counters, per-group
  // LayerNorm statistics partials of the residual stream
  float* bg_part = nullptr;
  unsigned* bg_cnt = nullptr;
  float* bg_spart = nullptr;
  float* bg_cen = nullptr;  // [2][16]: per-row centres of the folded LayerNorms' inputs
};

static void free_work(rtg_cache* c) {
  for (float** p : {&c->x, &c->ln, &c->qkv, &c->att, &c->h, &c->ws}) {
    if (*p) hipFree(*p);
    *p = nullptr;
  }
  c->rows_cap = 0;
  c->ws_floats = 0;
}

static void destroy_graph(rtg_cache* c) {
  if (c->graph_exec) hipGraphExecDestroy(c->graph_exec);
  if (c->graph) hipGraphDestroy(c->graph);
  c->graph_exec = nullptr;
  c->graph = nullptr;
}

static void ensure_rows(rtg_cache* c, size_t rows) {
  if (rows <= c->rows_cap) return;
  destroy_graph(c);
  free_work(c);
  const size_t d = c->m->cfg.n_embd;
  size_t cap = std::max<size_t>(rows, 16);
  HIPX(hipMalloc(&c->x, cap * d * 4));
  HIPX(hipMalloc(&c->ln, cap * d * 4));
  HIPX(hipMalloc(&c->qkv, cap * 3 * d * 4));
  HIPX(hipMalloc(&c->att, cap * d * 4));
  HIPX(hipMalloc(&c->h, cap * 4 * d * 4));
  // the split-k workspace for the largest need of the four layer GEMMs at
  // any row count up to cap (the split depends on the row blocks)
  size_t ws = 0;
  for (size_t r = 32; r < cap + 128; r += (r < 128 ? 32 : 128)) {
    const int M = (int)std::min(r, cap);
    for (const auto& nk : {std::make_pair(3 * d, d), std::make_pair(d, d), std::make_pair(4 * d, d),
                           std::make_pair(d, 4 * d)})
      ws = std::max(ws, gemm_splitk_ws_floats(M, (int)nk.first, (int)nk.second));
  }
  if (ws) HIPX(hipMalloc(&c->ws, ws * 4));
  c->ws_floats = ws;
  c->rows_cap = cap;
}

static void ensure_logits(rtg_cache* c, size_t rows) {
  if (rows <= c->logit_rows_cap) return;
  destroy_graph(c);
  if (c->pstate) persistent_state_destroy(c->pstate);  // it holds the logits pointer
  c->pstate = nullptr;
  if (c->logits) hipFree(c->logits);
  c->logits = nullptr;
  size_t cap = std::max<size_t>(rows, 16);
  HIPX(hipMalloc(&c->logits, cap * c->m->cfg.vocab_size * 4));
  c->logit_rows_cap = cap;
}

static rtg_cache* cache_create(const rtg_model* m, size_t batch) {
  std::unique_ptr<rtg_cache> c(new rtg_cache());
  c->m = m;
  c->batch = batch;
  const size_t L = m->cfg.n_layer, H = m->cfg.n_head, P = m->cfg.n_positions, hd = m->hd;
  c->layer_stride = batch * H * P * hd;
  try {
    HIPX(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    HIPX(hipMalloc(&c->k, std::max<size_t>(L * c->layer_stride, 1) * 4));
    HIPX(hipMalloc(&c->v, std::max<size_t>(L * c->layer_stride, 1) * 4));
    HIPX(hipMalloc(&c->pos_dev, 256));
    HIPX(hipMalloc(&c->step_dev, 256));
    HIPX(hipMalloc(&c->keys, std::max<size_t>(batch, 1) * 8));
    HIPX(hipMalloc(&c->token_dev, std::max<size_t>(batch, 1) * 4));
    HIPX(hipMalloc(&c->ids_dev, std::max<size_t>(batch * P, 1) * 4));
    HIPX(hipMalloc(&c->ids_in, std::max<size_t>(batch * P, 1) * 4));
    for (auto& e : c->ev) HIPX(hipEventCreate(&e));
    HIPX(hipMemsetAsync(c->pos_dev, 0, 256, c->stream));
    HIPX(hipMemsetAsync(c->step_dev, 0, 256, c->stream));
    launch_reset_keys(c->stream, (int)batch, c->keys);
    HIPX(hipStreamSynchronize(c->stream));
  } catch (...) {
    rtg_cache_destroy(c.release());
    throw;
  }
  return c.release();
}

rtg_model::~rtg_model() {
  for (auto& kv : pool) rtg_cache_destroy(kv.second);
  pool.clear();
  if (pplan) persistent_plan_destroy(pplan);
  if (rplan) rows_plan_destroy(rplan);
  if (arena) hipFree(arena);
}

// ---------------------------------------------------------------------------
// Pipelines
// ---------------------------------------------------------------------------

static KvDst kv_layer(const rtg_cache* c, size_t l) {
  KvDst kv;
  kv.k = c->k + l * c->layer_stride;
  kv.v = c->v + l * c->layer_stride;
  kv.n_head = (int)c->m->cfg.n_head;
  kv.n_pos = (int)c->m->cfg.n_positions;
  kv.d = (int)c->m->cfg.n_embd;
  return kv;
}

// Activation buffers of one forward pass: x, ln [M][d], qkv [M][3d],
// att [M][d], h [M][4d], the logits rows and the GEMMs' split-k workspace
// (ws_floats floats; null: the GEMMs run unsplit).
struct Work {
  float *x, *ln, *qkv, *att, *h, *logits;
  float* ws;
  size_t ws_floats;
};

static Work cache_work(const rtg_cache* c) {
  return Work{c->x, c->ln, c->qkv, c->att, c->h, c->logits, c->ws, c->ws_floats};
}

// forward_cached body for S sequences x T new tokens (gpt2.rs:376-396) on the
// MFMA prefill path, on the activation buffers w. ids_dev holds S*T ids;
// logits rows: all S*T (mode 0) or the last row of each sequence (mode 1,
// written as S rows).
static void enqueue_prefill(rtg_cache* c, const Work& w, const uint32_t* ids_dev, size_t S, size_t T, size_t past,
                            int logit_mode) {
  const rtg_model* m = c->m;
  const int d = (int)m->cfg.n_embd, V = (int)m->cfg.vocab_size, M = (int)(S * T);
  const float eps = m->cfg.layer_norm_epsilon;
  hipStream_t s = c->stream;
  launch_embed(s, m->wte, m->wtype, m->wpe, ids_dev, M, (int)T, (int)past, nullptr, d, w.x);
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const LayerW& L = m->layers[l];
    KvDst kv = kv_layer(c, l);
    launch_layernorm(s, w.x, L.ln1w, L.ln1b, eps, M, d, w.ln);
    launch_gemm_qkv(s, w.ln, d, L.wqkv, m->wtype, L.bqkv, w.qkv, 3 * d, M, d, (int)S, (int)T, (int)past, kv, w.ws,
                    w.ws_floats);
    launch_attn_prefill(s, w.qkv, (int)S, (int)T, (int)past, kv.k, kv.v, kv.n_head, kv.n_pos, d, w.att);
    launch_gemm(s, w.att, d, L.waproj, m->wtype, L.baproj, w.x, d, M, d, d, EPI_BIAS_RESID, w.ws, w.ws_floats);
    launch_layernorm(s, w.x, L.ln2w, L.ln2b, eps, M, d, w.ln);
    launch_gemm(s, w.ln, d, L.wfc, m->wtype, L.bfc, w.h, 4 * d, M, 4 * d, d, EPI_BIAS_GELU, w.ws, w.ws_floats);
    launch_gemm(s, w.h, 4 * d, L.wmproj, m->wtype, L.bmproj, w.x, d, M, d, 4 * d, EPI_BIAS_RESID, w.ws,
                w.ws_floats);
  }
  launch_layernorm(s, w.x, m->lnfw, m->lnfb, eps, M, d, w.ln);
  if (logit_mode == 0) {
    launch_gemm(s, w.ln, d, m->wte, m->wtype, nullptr, w.logits, V, M, V, d, EPI_NONE);
  } else {
    // Last row of each sequence: rows (s*T + T-1), stride T*d.
    launch_gemm(s, w.ln + (T - 1) * d, (int)(T * d), m->wte, m->wtype, nullptr, w.logits, V, (int)S, V, d,
                EPI_NONE);
  }
}

// ---- batched decode step on the tile-ordered GEMV (bgemv.h) ----

// The batched step needs every GEMV's K to be a whole number of k-tiles and at
// most 16 sequences; other shapes keep the per-op kernels below.
static bool batched_ok(const rtg_model* m, size_t B) {
  const size_t tk = m->wtype == W_F32 ? 16 : 32;
  // (the LayerNorm statistics of a row come in at most 128 panel groups)
  return B >= 1 && B <= 16 && m->cfg.n_embd % tk == 0 && m->cfg.n_embd <= 2048;
}

// Builds the model's tile-ordered weight copies and folded LayerNorm constants
// (once; callers may race, the mutex serialises them).
static const BatchedWeights* ensure_batched(const rtg_model* mc) {
  rtg_model* m = const_cast<rtg_model*>(mc);
  std::lock_guard<std::mutex> g(m->bw_mu);
  if (m->bw) return m->bw.get();
  const int d = (int)m->cfg.n_embd, V = (int)m->cfg.vocab_size, L = (int)m->layers.size(), wt = m->wtype;
  std::unique_ptr<BatchedWeights> bw(new BatchedWeights());
  const size_t tq = tiled_weight_bytes(3 * d, d, wt), tp = tiled_weight_bytes(d, d, wt);
  const size_t tf = tiled_weight_bytes(4 * d, d, wt), tm = tiled_weight_bytes(d, 4 * d, wt);
  const size_t tl = tiled_weight_bytes(V, d, wt);
  const size_t per_layer = align_up(tq, 256) + align_up(tp, 256) + align_up(tf, 256) + align_up(tm, 256);
  const size_t fold_layer = (size_t)(2 * 3 * d + 2 * 4 * d) * 4;
  const size_t total = per_layer * L + align_up(tl, 256) + align_up(fold_layer, 256) * L + align_up((size_t)2 * V * 4, 256);
  HIPX(hipDeviceSynchronize());
  HIPX(hipMalloc(&bw->arena, total));
  char* p = static_cast<char*>(bw->arena);
  auto take = [&](size_t n) {
    char* r = p;
    p += align_up(n, 256);
    return r;
  };
  auto tile = [&](const void* src, int N, int K, size_t bytes) {
    void* dst = take(bytes);
    if (!launch_tile_weights(nullptr, src, wt, N, K, dst)) throw HipError{"tile_weights launch failed"};
    return (const void*)dst;
  };
  for (int l = 0; l < L; ++l) {
    const LayerW& W = m->layers[l];
    BatchedWeights::Layer bl{};
    bl.qkv = tile(W.wqkv, 3 * d, d, tq);
    bl.proj = tile(W.waproj, d, d, tp);
    bl.fc = tile(W.wfc, 4 * d, d, tf);
    bl.mproj = tile(W.wmproj, d, 4 * d, tm);
    float* f = reinterpret_cast<float*>(take(fold_layer));
    float *sq = f, *cq = f + 3 * d, *sf = f + 6 * d, *cf = f + 10 * d;
    if (!ln_fold(W.wqkv, wt, 3 * d, d, W.ln1w, W.ln1b, W.bqkv, sq, cq) ||
        !ln_fold(W.wfc, wt, 4 * d, d, W.ln2w, W.ln2b, W.bfc, sf, cf))
      throw HipError{"ln_fold launch failed"};
    bl.sq = sq; bl.cq = cq; bl.sf = sf; bl.cf = cf;
    bw->layers.push_back(bl);
  }
  bw->lm = tile(m->wte, V, d, tl);
  float* fl = reinterpret_cast<float*>(take((size_t)2 * V * 4));
  if (!ln_fold(m->wte, wt, V, d, m->lnfw, m->lnfb, nullptr, fl, fl + V)) throw HipError{"ln_fold launch failed"};
  bw->sl = fl;
  bw->cl = fl + V;
  HIPX(hipDeviceSynchronize());
  bw->pq = bgemv_plan(3 * d, d, wt);
  bw->pp = bgemv_plan(d, d, wt);
  bw->pf = bgemv_plan(4 * d, d, wt);
  bw->pm = bgemv_plan(d, 4 * d, wt);
  bw->pl = bgemv_plan(V, d, wt);
  m->bw = std::move(bw);
  return m->bw.get();
}

// The cache's workspace for the batched step (allocated once per cache).
static void ensure_bg_work(rtg_cache* c, const BatchedWeights* bw) {
  if (c->bg_part) return;
  size_t part = 1, groups = 1;
  for (const BgemvPlan* pl : {&bw->pq, &bw->pp, &bw->pf, &bw->pm, &bw->pl}) {
    part = std::max(part, bgemv_work_floats(*pl));
    groups = std::max(groups, (size_t)pl->groups);
  }
  HIPX(hipMalloc(&c->bg_part, part * 4));
  HIPX(hipMalloc(&c->bg_cnt, groups * 4));
  HIPX(hipMalloc(&c->bg_spart, groups * 16 * 2 * 4));
  HIPX(hipMalloc(&c->bg_cen, 2 * 16 * 4));
  HIPX(hipMemsetAsync(c->bg_cnt, 0, groups * 4, c->stream));
  HIPX(hipStreamSynchronize(c->stream));
}

// Prepares the decode step of a cache without a batch-1 persistent state
// (before any capture): the batched weights and the step's workspace.
static void prepare_decode(rtg_cache* c) {
  if (c->pstate || !batched_ok(c->m, c->batch)) return;
  ensure_bg_work(c, ensure_batched(c->m));
}

// One decode step for B sequences: per layer four tile-ordered GEMVs with
// LayerNorm folded into c_attn / c_fc / the LM head (row statistics written by
// the residual epilogues) and the cached attention; forward_cached with one
// token per sequence (gpt2.rs:376-396, 477-538).
static void enqueue_decode_step_batched(rtg_cache* c) {
  const rtg_model* m = c->m;
  const BatchedWeights* bw = m->bw.get();
  const int d = (int)m->cfg.n_embd, V = (int)m->cfg.vocab_size, B = (int)c->batch;
  const float eps = m->cfg.layer_norm_epsilon;
  hipStream_t s = c->stream;
  auto base = [&]() {
    BgemvArgs a{};
    a.M = B;
    a.wtype = m->wtype;
    a.part = c->bg_part;
    a.cnt = c->bg_cnt;
    a.eps = eps;
    return a;
  };
  auto run = [&](const BgemvPlan& pl, const BgemvArgs& a) {
    if (!launch_bgemv(s, pl, a)) throw HipError{"bgemv launch failed"};
  };
  // c->ln holds x scaled by the gain of the LayerNorm folded into the next
  // GEMV (written by the embedding and by each residual epilogue); c->ln,
  // c->att and c->h are in the GEMV input layout (xt_index, tile width tk)
  const int tk = m->wtype == W_F32 ? 16 : 32;
  const size_t NL = m->layers.size();
  // Centres of the folded LayerNorms (two alternating per-row buffers): the
  // GEMV input c->ln holds (x - cen_cur) * g; each LayerNorm-folded GEMV
  // writes its rows' exact mean into the other buffer, and the residual
  // epilogue after it centres the next input on that mean, so the fold only
  // ever subtracts the drift of the mean between two LayerNorms.
  float* cen_cur = c->bg_cen;
  float* cen_next = c->bg_cen + 16;
  if (!launch_embed_stats(s, m->wte, m->wtype, m->wpe, c->token_dev, c->pos_dev, B, d, c->x, c->bg_spart,
                          NL ? m->layers[0].ln1w : m->lnfw, c->ln, cen_cur))
    throw HipError{"embed_stats launch failed"};
  // shape of the statistics partials the last residual writer left
  int st_groups = 1, st_cols = d;
  auto ln_in = [&](BgemvArgs& a, const float* g, const float* sv, bool record) {
    a.ln_g = g; a.ln_s = sv; a.ln_part = c->bg_spart; a.ln_groups = st_groups; a.ln_cols = st_cols;
    a.cen_in = cen_cur;
    if (record) {
      cen_next = cen_cur == c->bg_cen ? c->bg_cen + 16 : c->bg_cen;
      a.cen_out = cen_next;
    }
  };
  auto resid_out = [&](BgemvArgs& a, const BgemvPlan& pl, const float* g_next) {
    a.stats_part = c->bg_spart;
    a.xg = c->ln;
    a.g_next = g_next;
    a.xg_cen = cen_next;
    cen_cur = cen_next;
    st_groups = pl.groups;
    st_cols = 16 * pl.npw;
  };
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const LayerW& L = m->layers[l];
    const BatchedWeights::Layer& T = bw->layers[l];
    KvDst kv = kv_layer(c, l);
    {  // LN1 + c_attn; k/v of the new token into the cache
      BgemvArgs a = base();
      a.X = c->ln; a.Wt = T.qkv; a.N = 3 * d; a.K = d; a.bias = T.cq;
      ln_in(a, L.ln1w, T.sq, true);
      a.epi = EPI_BIAS;
      a.qkv = BgemvQkv{c->qkv, d, d, kv, c->pos_dev};
      run(bw->pq, a);
    }
    launch_attn_decode(s, B, c->qkv, d, kv.k, kv.v, kv.n_head, kv.n_pos, c->pos_dev, c->att, d, tk);
    {  // attention c_proj + residual; statistics partials for LN2
      BgemvArgs a = base();
      a.X = c->att; a.Wt = T.proj; a.N = d; a.K = d; a.bias = L.baproj;
      a.C = c->x; a.ldc = d; a.epi = EPI_BIAS_RESID;
      resid_out(a, bw->pp, L.ln2w);
      run(bw->pp, a);
    }
    {  // LN2 + c_fc + gelu_new
      BgemvArgs a = base();
      a.X = c->ln; a.Wt = T.fc; a.N = 4 * d; a.K = d; a.bias = T.cf;
      ln_in(a, L.ln2w, T.sf, true);
      a.C = c->h; a.c_tiled = true; a.epi = EPI_BIAS_GELU;
      run(bw->pf, a);
    }
    {  // mlp c_proj + residual; statistics partials for the next LayerNorm
      BgemvArgs a = base();
      a.X = c->h; a.Wt = T.mproj; a.N = d; a.K = 4 * d; a.bias = L.bmproj;
      a.C = c->x; a.ldc = d; a.epi = EPI_BIAS_RESID;
      resid_out(a, bw->pm, l + 1 < NL ? m->layers[l + 1].ln1w : m->lnfw);
      run(bw->pm, a);
    }
  }
  {  // ln_f + tied LM head (gpt2.rs:392-396)
    BgemvArgs a = base();
    a.X = c->ln; a.Wt = bw->lm; a.N = V; a.K = d; a.bias = bw->cl;
    ln_in(a, m->lnfw, bw->sl, false);
    a.C = c->logits; a.ldc = V; a.epi = EPI_BIAS;
    run(bw->pl, a);
  }
  // (the argmax in the LM head's epilogue, a per-row atomic max per
  // workgroup, was measured slower than this separate kernel)
  launch_argmax(s, c->logits, V, B, V, c->keys);
}

// One decode step for all B sequences of the cache, reading the token from
// token_dev and the position from pos_dev (both device-resident), writing the
// argmax token back to token_dev and ids_dev[b][step]. Capturable.
static void enqueue_decode_step(rtg_cache* c, int pos = -1) {
  const rtg_model* m = c->m;
  const int d = (int)m->cfg.n_embd, V = (int)m->cfg.vocab_size, B = (int)c->batch;
  const float eps = m->cfg.layer_norm_epsilon;
  hipStream_t s = c->stream;
  const int P = (int)m->cfg.n_positions;
  if (c->pstate) {
    HIPX(persistent_decode_step(c->pstate, s, /*cooperative=*/false, pos));
  } else if (c->bg_part) {
    enqueue_decode_step_batched(c);
  } else {
    launch_embed(s, m->wte, m->wtype, m->wpe, c->token_dev, B, 1, 0, c->pos_dev, d, c->x);
    for (size_t l = 0; l < m->layers.size(); ++l) {
      const LayerW& L = m->layers[l];
      KvDst kv = kv_layer(c, l);
      launch_layernorm(s, c->x, L.ln1w, L.ln1b, eps, B, d, c->ln);
      launch_gemv_qkv(s, B, L.wqkv, m->wtype, L.bqkv, c->ln, d, c->qkv, d, d, kv, c->pos_dev);
      launch_attn_decode(s, B, c->qkv, d, kv.k, kv.v, kv.n_head, kv.n_pos, c->pos_dev, c->att, d);
      launch_gemv(s, B, L.waproj, m->wtype, L.baproj, c->att, d, c->x, d, d, d, EPI_BIAS_RESID);
      launch_layernorm(s, c->x, L.ln2w, L.ln2b, eps, B, d, c->ln);
      launch_gemv(s, B, L.wfc, m->wtype, L.bfc, c->ln, d, c->h, 4 * d, 4 * d, d, EPI_BIAS_GELU);
      launch_gemv(s, B, L.wmproj, m->wtype, L.bmproj, c->h, 4 * d, c->x, d, d, 4 * d, EPI_BIAS_RESID);
    }
    launch_layernorm(s, c->x, m->lnfw, m->lnfb, eps, B, d, c->ln);
    launch_gemv(s, B, m->wte, m->wtype, nullptr, c->ln, d, c->logits, V, V, d, EPI_NONE);
    launch_argmax(s, c->logits, V, B, V, c->keys);
  }
  if (!c->pstate)  // the persistent step finishes itself
    launch_finalize(s, B, c->keys, c->token_dev, c->ids_dev, P, c->pos_dev, c->step_dev, nullptr);
}

// Device-side fills (no staging copy of a host value); never captured.
static void set_counters(rtg_cache* c, int pos, int step) {
  HIPX(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(c->pos_dev), pos, 1, c->stream));
  HIPX(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(c->step_dev), step, 1, c->stream));
}

// The multi-row forward runs S sequences x T tokens of a cache of batch S in
// one launch (RTG_NO_ROWS=1: the per-op prefill kernels instead).
static bool rows_path(const rtg_cache* c, size_t S, size_t T) {
  const char* off = getenv("RTG_NO_ROWS");
  if (off && off[0] == '1') return false;
  return c->m->rplan && S == c->batch && rows_supported(c->m->rplan, (int)S, (int)T);
}

// Enqueues the multi-row forward on the cache's stream (the caller holds
// persistent_launch_lock until the stream drains): ids_dev [S*T] at position
// past, logits [S*T][V]; state st (default: the cache's own, made on first use).
static void enqueue_rows(rtg_cache* c, const uint32_t* ids_dev, size_t S, size_t T, size_t past, float* logits,
                         RowsState* st = nullptr, const RowsFinish* fin = nullptr) {
  const rtg_model* m = c->m;
  if (!st) {
    if (!c->rstate) {
      c->rstate = rows_state_create(m->rplan);
      if (!c->rstate) throw HipError{"multi-row forward: state allocation failed"};
    }
    st = c->rstate;
  }
  HIPX(rows_forward(m->rplan, st, c->stream, c->k, c->v, (long)c->layer_stride, ids_dev, (int)S, (int)T, (int)past,
                    nullptr, logits, fin));
}

// After the stream has drained: a bounded wait of the multi-row forward that
// timed out becomes an error (its word is cleared for the next launch).
static void check_rows(RowsState* st) {
  rows_dump_trace();
  unsigned e = 0;
  HIPX(hipMemcpy(&e, rows_err(st), 4, hipMemcpyDeviceToHost));
  if (e) {
    HIPX(hipMemset(rows_err(st), 0, 4));
    throw HipError{fmt("multi-row forward timed out waiting for a peer (phase %u)", e)};
  }
}

static void ensure_graph(rtg_cache* c) {
  if (c->graph_exec) return;
  HIPX(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  enqueue_decode_step(c);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  HIPX(e);
  c->graph = g;
  HIPX(hipGraphInstantiate(&c->graph_exec, c->graph, nullptr, nullptr, 0));
}

// ---------------------------------------------------------------------------
// Validation shared by the entry points (gpt2.rs:364-377, 616-618)
// ---------------------------------------------------------------------------

static std::string check_ids(const rtg_model* m, const uint32_t* ids, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (ids[i] >= m->cfg.vocab_size)
      return fmt("Token ID %zu out of range (vocab_size=%zu)", (size_t)ids[i], m->cfg.vocab_size);
  return "";
}

static std::string check_cached(const rtg_model* m, size_t past, const uint32_t* ids, size_t n) {
  if (n == 0) return "Empty input";
  const size_t total = past + n;
  if (total > m->cfg.n_positions)
    return fmt("Total sequence length %zu exceeds max position %zu", total, m->cfg.n_positions);
  return check_ids(m, ids, n);
}

// forward_cached for all sequences of a cache: ids [B][n].
static void forward_cached_impl(rtg_cache* c, const uint32_t* ids, size_t n, float* logits_out) {
  const rtg_model* m = c->m;
  const size_t B = c->batch, V = m->cfg.vocab_size;
  ensure_rows(c, B * n);
  ensure_logits(c, B * n);
  if (n == 1 && B == 1 && persistent_supported(m->pplan, 1)) {
    // one new token at batch 1: the persistent decode step, the kernel
    // generate_cached runs per token; its token is read from token_dev at
    // position *pos_dev = past, its logits land in c->logits
    if (!c->pstate) {
      c->pstate = persistent_state_create(m->pplan, c->k, c->v, 1, c->token_dev, c->pos_dev, c->logits, c->keys,
                                          c->ids_dev, c->step_dev);
      destroy_graph(c);
    }
  }
  if (n == 1 && B == 1 && c->pstate) {
    std::lock_guard<std::mutex> plock(persistent_launch_lock(m->device));
    HIPX(hipMemcpyAsync(c->token_dev, ids, 4, hipMemcpyHostToDevice, c->stream));
    set_counters(c, (int)c->len, 0);
    HIPX(persistent_decode_step(c->pstate, c->stream, /*cooperative=*/false, (int)c->len));
    if (logits_out) HIPX(hipMemcpyAsync(logits_out, c->logits, V * 4, hipMemcpyDeviceToHost, c->stream));
    HIPX(hipStreamSynchronize(c->stream));
    unsigned e = 0;
    HIPX(hipMemcpy(&e, persistent_err(c->pstate), 4, hipMemcpyDeviceToHost));
    if (e) {
      HIPX(hipMemset(persistent_err(c->pstate), 0, 4));
      throw HipError{fmt("persistent decode step timed out waiting for a peer (code %u)", e)};
    }
    c->len += 1;
    return;
  }
  if (n == 1 && B >= 2 && !c->pstate && batched_ok(m, B)) {
    // one new token per sequence: the batched decode step (the same kernels
    // generate_cached_batched replays), its token read from token_dev at
    // position *pos_dev = past
    prepare_decode(c);
    HIPX(hipMemcpyAsync(c->token_dev, ids, B * 4, hipMemcpyHostToDevice, c->stream));
    set_counters(c, (int)c->len, 0);
    enqueue_decode_step(c);
  } else if (rows_path(c, B, n)) {
    std::lock_guard<std::mutex> plock(persistent_launch_lock(m->device));
    HIPX(hipMemcpyAsync(c->ids_in, ids, B * n * 4, hipMemcpyHostToDevice, c->stream));
    enqueue_rows(c, c->ids_in, B, n, c->len, c->logits);
    if (logits_out) HIPX(hipMemcpyAsync(logits_out, c->logits, B * n * V * 4, hipMemcpyDeviceToHost, c->stream));
    HIPX(hipStreamSynchronize(c->stream));
    check_rows(c->rstate);
    c->len += n;
    return;
  } else {
    HIPX(hipMemcpyAsync(c->ids_in, ids, B * n * 4, hipMemcpyHostToDevice, c->stream));
    enqueue_prefill(c, cache_work(c), c->ids_in, B, n, c->len, 0);
  }
  if (logits_out) HIPX(hipMemcpyAsync(logits_out, c->logits, B * n * V * 4, hipMemcpyDeviceToHost, c->stream));
  HIPX(hipStreamSynchronize(c->stream));
  c->len += n;
}

static rtg_cache* pool_take(const rtg_model* mc, size_t batch) {
  rtg_model* m = const_cast<rtg_model*>(mc);
  {
    std::lock_guard<std::mutex> g(m->pool_mu);
    auto it = m->pool.find(batch);
    if (it != m->pool.end()) {
      rtg_cache* c = it->second;
      m->pool.erase(it);
      c->len = 0;
      return c;
    }
  }
  return cache_create(mc, batch);
}

static void pool_give(const rtg_model* mc, rtg_cache* c) {
  rtg_model* m = const_cast<rtg_model*>(mc);
  std::lock_guard<std::mutex> g(m->pool_mu);
  m->pool.emplace(c->batch, c);
}

struct PoolLease {
  const rtg_model* m;
  rtg_cache* c;
  PoolLease(const rtg_model* mm, size_t b) : m(mm), c(pool_take(mm, b)) {}
  ~PoolLease() {
    if (c) pool_give(m, c);
  }
};

// generate_cached over B equal-length prompts (gpt2.rs:405-441), greedy or,
// with sp (B = 1), choosing every token with the device sampler
// (sample_logits, gpt2.rs:871-906): the whole loop stays on the device.
static void generate_greedy(const rtg_model* m, const uint32_t* prompts, size_t B, size_t n, size_t max_new,
                            uint32_t* out, rtg_timing* timing, const SampleParams* sp = nullptr) {
  PoolLease lease(m, B);
  rtg_cache* c = lease.c;
  const size_t V = m->cfg.vocab_size, P = m->cfg.n_positions;
  const size_t steps = max_new > 0 ? max_new : 1;  // first token comes from prefill
  ensure_rows(c, B * n);
  ensure_logits(c, B * n);
  hipStream_t s = c->stream;
  // overwrite the argmax token of the step just enqueued with the sampler's choice
  auto sample = [&](const float* row) {
    if (sp && !launch_sample(s, row, (int)V, c->ids_in, (int)n, c->ids_dev, c->step_dev, *sp, c->token_dev))
      throw HipError{"vocabulary too large for the device sampler"};
  };
  if (!c->pstate && persistent_supported(m->pplan, (int)B)) {
    c->pstate = persistent_state_create(m->pplan, c->k, c->v, (int)B, c->token_dev, c->pos_dev, c->logits, c->keys,
                                        c->ids_dev, c->step_dev);
    destroy_graph(c);  // the step graph changes shape
  }
  prepare_decode(c);
  // The persistent step's workgroups wait on each other: no second persistent
  // step of this process may be in flight on the device (another thread's
  // cache) until this stream has drained.
  const bool rows = rows_path(c, B, n);
  if (rows && !c->rstate) {  // (allocated before the timed prefill)
    c->rstate = rows_state_create(m->rplan);
    if (!c->rstate) throw HipError{"multi-row forward: state allocation failed"};
  }
  std::unique_lock<std::mutex> plock;
  if (c->pstate || rows) plock = std::unique_lock<std::mutex>(persistent_launch_lock(m->device));
  HIPX(hipMemcpyAsync(c->ids_in, prompts, B * n * 4, hipMemcpyHostToDevice, s));
  HIPX(hipEventRecord(c->ev[0], s));
  // finalize advances pos by one: after it, pos = n, the position of the
  // prefill token that the first decode step consumes.
  set_counters(c, (int)n - 1, 0);
  if (rows) {
    // the prefill with the argmax of each sequence's last row and the
    // finalize in the same launch
    const RowsFinish fin{c->keys, c->token_dev, c->ids_dev, (int)P, c->pos_dev, c->step_dev};
    enqueue_rows(c, c->ids_in, B, n, 0, c->logits, nullptr, &fin);
  } else {
    enqueue_prefill(c, cache_work(c), c->ids_in, B, n, 0, 0);
    // argmax of the last row of each sequence (extract_row(logits, n-1))
    launch_argmax(s, c->logits + (n - 1) * V, (long)(n * V), (int)B, (int)V, c->keys);
    launch_finalize(s, (int)B, c->keys, c->token_dev, c->ids_dev, (int)P, c->pos_dev, c->step_dev);
  }
  sample(c->logits + (n - 1) * V);
  HIPX(hipEventRecord(c->ev[1], s));
  // The persistent step (one kernel) is launched directly: replaying it as a
  // one-node graph was measured to leave ~8 us between launches instead of ~1.
  // RTG_NO_GRAPH=1 does the same for the batched step's kernels (for
  // per-kernel profiling; same results).
  const char* ng = getenv("RTG_NO_GRAPH");
  if (c->pstate || (ng && ng[0] == '1')) {
    for (size_t i = 1; i < steps; ++i) {
      enqueue_decode_step(c, (int)(n + i - 1));  // step i consumes the token at position n + i - 1
      sample(c->logits);
    }
  } else {
    ensure_graph(c);
    for (size_t i = 1; i < steps; ++i) {
      HIPX(hipGraphLaunch(c->graph_exec, s));
      sample(c->logits);
    }
  }
  HIPX(hipEventRecord(c->ev[2], s));
  // Optional profiling pass: rewind to the first decode step and replay the
  // steps launch by launch with events around the persistent kernel. Inputs
  // (tokens, positions, cache rows) are the same, so are the results.
  double kern_ms = 0.0;
  size_t kern_n = 0;
  if (timing && timing->profile_kernels && c->pstate && steps > 1 && !sp) {
    std::vector<hipEvent_t> evs(2 * (steps - 1));
    for (auto& e : evs) HIPX(hipEventCreate(&e));
    set_counters(c, (int)n, 1);
    HIPX(hipMemcpyAsync(c->token_dev, c->ids_dev, 4, hipMemcpyDeviceToDevice, s));
    for (size_t i = 1; i < steps; ++i) {
      HIPX(hipEventRecord(evs[2 * (i - 1)], s));
      HIPX(persistent_decode_step(c->pstate, s, /*cooperative=*/true, (int)(n + i - 1)));
      HIPX(hipEventRecord(evs[2 * (i - 1) + 1], s));
    }
    HIPX(hipStreamSynchronize(s));
    for (size_t i = 0; i + 1 < evs.size(); i += 2) {
      float ms = 0.f;
      HIPX(hipEventElapsedTime(&ms, evs[i], evs[i + 1]));
      kern_ms += ms;
      ++kern_n;
    }
    for (auto& e : evs) hipEventDestroy(e);
  }
  std::vector<uint32_t> gen(B * P);
  HIPX(hipMemcpyAsync(gen.data(), c->ids_dev, B * P * 4, hipMemcpyDeviceToHost, s));
  HIPX(hipStreamSynchronize(s));
  if (rows) check_rows(c->rstate);
  if (c->pstate) {
    persistent_dump_trace(c->pstate);
    unsigned e = 0;
    HIPX(hipMemcpy(&e, persistent_err(c->pstate), 4, hipMemcpyDeviceToHost));
    if (e) {
      HIPX(hipMemset(persistent_err(c->pstate), 0, 4));
      throw HipError{fmt("persistent decode step timed out waiting for a peer (code %u)", e)};
    }
  }
  c->len = n + steps - 1;  // the last generated token is never fed back
  const size_t outlen = n + steps;
  for (size_t b = 0; b < B; ++b) {
    memcpy(out + b * outlen, prompts + b * n, n * 4);
    memcpy(out + b * outlen + n, gen.data() + b * P, steps * 4);
  }
  if (timing) {
    float a = 0.f, b2 = 0.f;
    HIPX(hipEventElapsedTime(&a, c->ev[0], c->ev[1]));
    HIPX(hipEventElapsedTime(&b2, c->ev[1], c->ev[2]));
    timing->prefill_ms = a;
    timing->decode_ms = b2;
    timing->decode_steps = steps - 1;
    timing->decode_kernel_ms = kern_ms;
    timing->decode_kernel_launches = kern_n;
  }
}

// ---------------------------------------------------------------------------
// Model construction (gpt2.rs:214-263)
// ---------------------------------------------------------------------------

namespace {
// A weight as the caller or the file holds it: f32, bf16 or f16 elements
// (uploaded as they are and converted on the device), or an f32 decode on the
// host of any other element type.
struct HostTensor {
  std::vector<size_t> shape;
  const void* data = nullptr;
  int stype = SRC_F32;
  std::vector<float> owned;
  size_t numel() const {
    size_t n = 1;
    for (size_t x : shape) n *= x;
    return n;
  }
  size_t bytes() const { return numel() * (stype == SRC_F32 ? 4 : 2); }
};

using Lookup = std::map<std::string, HostTensor>;

std::string shape_str(const std::vector<size_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

rtg_result build_model(const rtg_config* cfg, Lookup& lk, rtg_storage storage, rtg_model** out) {
  const size_t d = cfg->n_embd, L = cfg->n_layer, V = cfg->vocab_size, P = cfg->n_positions, H = cfg->n_head;
  // gpt2.rs:224-263: look up every name first, in the reference's order.
  std::vector<std::string> names = {"wte.weight", "wpe.weight", "ln_f.weight", "ln_f.bias"};
  const char* per[] = {"ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
                       "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
                       "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight", "mlp.c_proj.bias"};
  for (size_t i = 0; i < L; ++i)
    for (const char* p : per) names.push_back("h." + std::to_string(i) + "." + p);
  for (const auto& nm : names)
    if (!lk.count(nm)) return err("Missing weight: " + nm);
  if (H == 0 || d == 0 || d % H != 0) return err(fmt("n_embd %zu is not divisible by n_head %zu", d, H));
  const size_t hd = d / H;
  if (hd > 64) return err(fmt("head_dim %zu > 64 is not supported", hd));
  if (d % 8 != 0) return err(fmt("n_embd %zu must be a multiple of 8", d));
  // Shapes (the reference does not check them; a mismatch there is a panic or garbage).
  auto want = [&](const std::string& nm, std::vector<size_t> s) -> std::string {
    const auto& t = lk[nm];
    if (t.shape != s) return "Shape mismatch for " + nm + ": expected " + shape_str(s) + ", got " + shape_str(t.shape);
    return "";
  };
  std::string e;
  if (!(e = want("wte.weight", {V, d})).empty() || !(e = want("wpe.weight", {P, d})).empty() ||
      !(e = want("ln_f.weight", {d})).empty() || !(e = want("ln_f.bias", {d})).empty())
    return err(e);
  for (size_t i = 0; i < L; ++i) {
    std::string p = "h." + std::to_string(i) + ".";
    std::vector<std::pair<const char*, std::vector<size_t>>> sh = {
        {"ln_1.weight", {d}}, {"ln_1.bias", {d}}, {"attn.c_attn.weight", {d, 3 * d}}, {"attn.c_attn.bias", {3 * d}},
        {"attn.c_proj.weight", {d, d}}, {"attn.c_proj.bias", {d}}, {"ln_2.weight", {d}}, {"ln_2.bias", {d}},
        {"mlp.c_fc.weight", {d, 4 * d}}, {"mlp.c_fc.bias", {4 * d}}, {"mlp.c_proj.weight", {4 * d, d}},
        {"mlp.c_proj.bias", {d}}};
    for (auto& kv : sh)
      if (!(e = want(p + kv.first, kv.second)).empty()) return err(e);
  }
  std::string derr = check_device();
  if (!derr.empty()) return err(derr);

  std::unique_ptr<rtg_model> m(new rtg_model());
  m->cfg = *cfg;
  m->hd = (int)hd;
  m->wtype = storage == RTG_STORE_BF16 ? W_BF16 : W_F32;
  hipGetDevice(&m->device);
  const size_t wb = m->wtype == W_BF16 ? 2 : 4;
  // Arena layout: per layer [wqkv wproj wfc wmproj | biases | LN], then wte, wpe, ln_f.
  std::vector<size_t> offs;
  size_t cur = 0;
  auto take = [&](size_t bytes) {
    size_t o = cur;
    cur = align_up(cur + bytes, 256);
    return o;
  };
  struct LOff {
    size_t wqkv, waproj, wfc, wmproj, bqkv, baproj, bfc, bmproj, ln1w, ln1b, ln2w, ln2b;
  };
  std::vector<LOff> lo(L);
  for (size_t i = 0; i < L; ++i) {
    lo[i].wqkv = take(3 * d * d * wb);
    lo[i].waproj = take(d * d * wb);
    lo[i].wfc = take(4 * d * d * wb);
    lo[i].wmproj = take(4 * d * d * wb);
    lo[i].bqkv = take(3 * d * 4);
    lo[i].baproj = take(d * 4);
    lo[i].bfc = take(4 * d * 4);
    lo[i].bmproj = take(d * 4);
    lo[i].ln1w = take(d * 4);
    lo[i].ln1b = take(d * 4);
    lo[i].ln2w = take(d * 4);
    lo[i].ln2b = take(d * 4);
  }
  const size_t o_wte = take(V * d * wb), o_wpe = take(P * d * 4), o_lnfw = take(d * 4), o_lnfb = take(d * 4);
  float* staging = nullptr;
  try {
    HIPX(hipMalloc(&m->arena, cur));
    m->arena_bytes = cur;
    char* A = reinterpret_cast<char*>(m->arena);
    size_t stage_max = std::max({V * d, P * d, 4 * d * d});
    HIPX(hipMalloc(&staging, stage_max * 4));
    hipStream_t s = nullptr;
    // Tensors go to the device in their own element type; widening,
    // narrowing to the storage type and the transpose run there.
    auto upload_f32 = [&](const std::string& nm, size_t off) {
      const auto& t = lk[nm];
      if (t.stype == SRC_F32) {
        HIPX(hipMemcpy(A + off, t.data, t.bytes(), hipMemcpyHostToDevice));
        return;
      }
      HIPX(hipMemcpy(staging, t.data, t.bytes(), hipMemcpyHostToDevice));
      launch_convert_to(s, staging, t.stype, (long)t.numel(), A + off, W_F32);
      HIPX(hipGetLastError());
      HIPX(hipDeviceSynchronize());
    };
    auto upload_wt = [&](const std::string& nm, size_t off) {  // [K][N] -> W^T [N][K] in storage type
      const auto& t = lk[nm];
      const size_t K = t.shape[0], N = t.shape[1];
      HIPX(hipMemcpy(staging, t.data, t.bytes(), hipMemcpyHostToDevice));
      launch_transpose_to(s, staging, t.stype, (int)K, (int)N, A + off, m->wtype);
      HIPX(hipGetLastError());
      HIPX(hipDeviceSynchronize());
    };
    m->layers.resize(L);
    for (size_t i = 0; i < L; ++i) {
      std::string p = "h." + std::to_string(i) + ".";
      upload_wt(p + "attn.c_attn.weight", lo[i].wqkv);
      upload_wt(p + "attn.c_proj.weight", lo[i].waproj);
      upload_wt(p + "mlp.c_fc.weight", lo[i].wfc);
      upload_wt(p + "mlp.c_proj.weight", lo[i].wmproj);
      upload_f32(p + "attn.c_attn.bias", lo[i].bqkv);
      upload_f32(p + "attn.c_proj.bias", lo[i].baproj);
      upload_f32(p + "mlp.c_fc.bias", lo[i].bfc);
      upload_f32(p + "mlp.c_proj.bias", lo[i].bmproj);
      upload_f32(p + "ln_1.weight", lo[i].ln1w);
      upload_f32(p + "ln_1.bias", lo[i].ln1b);
      upload_f32(p + "ln_2.weight", lo[i].ln2w);
      upload_f32(p + "ln_2.bias", lo[i].ln2b);
      LayerW& w = m->layers[i];
      w.wqkv = A + lo[i].wqkv;
      w.waproj = A + lo[i].waproj;
      w.wfc = A + lo[i].wfc;
      w.wmproj = A + lo[i].wmproj;
      w.bqkv = reinterpret_cast<float*>(A + lo[i].bqkv);
      w.baproj = reinterpret_cast<float*>(A + lo[i].baproj);
      w.bfc = reinterpret_cast<float*>(A + lo[i].bfc);
      w.bmproj = reinterpret_cast<float*>(A + lo[i].bmproj);
      w.ln1w = reinterpret_cast<float*>(A + lo[i].ln1w);
      w.ln1b = reinterpret_cast<float*>(A + lo[i].ln1b);
      w.ln2w = reinterpret_cast<float*>(A + lo[i].ln2w);
      w.ln2b = reinterpret_cast<float*>(A + lo[i].ln2b);
    }
    {
      const auto& t = lk["wte.weight"];
      HIPX(hipMemcpy(staging, t.data, t.bytes(), hipMemcpyHostToDevice));
      launch_convert_to(s, staging, t.stype, (long)(V * d), A + o_wte, m->wtype);
      HIPX(hipGetLastError());
      HIPX(hipDeviceSynchronize());
    }
    upload_f32("wpe.weight", o_wpe);
    upload_f32("ln_f.weight", o_lnfw);
    upload_f32("ln_f.bias", o_lnfb);
    m->wte = A + o_wte;
    m->wpe = reinterpret_cast<float*>(A + o_wpe);
    m->lnfw = reinterpret_cast<float*>(A + o_lnfw);
    m->lnfb = reinterpret_cast<float*>(A + o_lnfb);
    HIPX(hipFree(staging));
    staging = nullptr;
  } catch (const HipError& he) {
    if (staging) hipFree(staging);
    return err(he.msg);  } catch (const std::exception& ex) {
    if (staging) hipFree(staging);
    return err_internal(ex);
  }
  size_t np = V * d + P * d + 2 * d;
  np += L * (2 * d + d * 3 * d + 3 * d + d * d + d + 2 * d + d * 4 * d + 4 * d + 4 * d * d + d);
  m->nparams = np;
  {
    PersistentWeights pw;
    pw.cfg = m->cfg;
    pw.wtype = m->wtype;
    pw.wte = m->wte;
    pw.wpe = m->wpe;
    pw.lnfw = m->lnfw;
    pw.lnfb = m->lnfb;
    for (auto& l : m->layers)
      pw.layers.push_back({l.wqkv, l.waproj, l.wfc, l.wmproj, l.bqkv, l.baproj, l.bfc, l.bmproj, l.ln1w, l.ln1b,
                           l.ln2w, l.ln2b});
    m->pplan = persistent_plan_create(pw);
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      m->rplan = rows_plan_create(pw, cus);
  }
  *out = m.release();
  return ok();
}

bool decode_f64(const void* data, size_t n, std::vector<float>* out) {
  out->resize(n);
  const uint8_t* raw = reinterpret_cast<const uint8_t*>(data);
  for (size_t i = 0; i < n; ++i) {
    double v;
    memcpy(&v, raw + 8 * i, 8);
    (*out)[i] = (float)v;
  }
  return true;
}
}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" {

void rtg_init(void) { hipInit(0); }
void rtg_cleanup(void) {}
const char* rtg_version(void) { return "rtgpu 0.1.0 (gfx950)"; }

void rtg_free_error_message(char* msg) { free(msg); }

rtg_result rtg_model_from_host(const rtg_config* cfg, const rtg_named_tensor* tensors, size_t n, rtg_storage storage,
                               rtg_model** out) {
  try {
    if (!cfg || !out) return err("null argument");
    Lookup lk;
    for (size_t i = 0; i < n; ++i) {
      const rtg_named_tensor& t = tensors[i];
      HostTensor& h = lk[t.name];
      h.shape.assign(t.shape, t.shape + t.ndim);
      switch (t.dtype) {
        case RTG_F32: h.stype = SRC_F32; h.data = t.data; break;
        case RTG_BF16: h.stype = SRC_BF16; h.data = t.data; break;
        case RTG_F16: h.stype = SRC_F16; h.data = t.data; break;
        case RTG_F64:
          decode_f64(t.data, h.numel(), &h.owned);
          h.stype = SRC_F32;
          h.data = h.owned.data();
          break;
        default: return err("Unsupported dtype for " + std::string(t.name));
      }
    }
    return build_model(cfg, lk, storage, out);
  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
}

rtg_result rtg_model_from_safetensors(const char* path, const rtg_config* cfg, rtg_storage storage,
                                      rtg_model** out) {
  try {
    if (!cfg || !out || !path) return err("null argument");
    StFile f;
    std::string e = st_read_file(path, &f);
    if (!e.empty()) return err("Failed to load safetensors: " + e);
    // F32, BF16 and F16 tensors are used in place in the mapping (no host copy);
    // other element types are decoded to f32 (safetensors.rs:232-348).
    Lookup lk;
    for (auto& kv : f.entries) {
      const StEntry& en = kv.second;
      HostTensor& h = lk[kv.first];
      h.shape = en.shape;
      if (en.dtype == "F32" || en.dtype == "BF16" || en.dtype == "F16") {
        e = st_check_size(en, en.dtype == "F32" ? 4 : 2, en.dtype.c_str());
        h.stype = en.dtype == "F32" ? SRC_F32 : en.dtype == "BF16" ? SRC_BF16 : SRC_F16;
        h.data = st_data(f, en);
      } else {
        e = st_decode_f32(f, en, &h.owned);
        h.stype = SRC_F32;
        h.data = h.owned.data();
      }
      if (!e.empty()) return err("Failed to load safetensors: " + e);
    }
    return build_model(cfg, lk, storage, out);
  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
}

void rtg_model_destroy(rtg_model* model) { delete model; }

size_t rtg_num_parameters(const rtg_model* model) { return model ? model->nparams : 0; }

rtg_result rtg_cache_new(const rtg_model* model, size_t batch, rtg_cache** out) {
  if (!model || !out) return err("null argument");
  if (batch == 0) return err("batch must be >= 1");
  try {
    *out = cache_create(model, batch);
  } catch (const HipError& e) {
    return err(e.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

size_t rtg_cache_len(const rtg_cache* cache) { return cache ? cache->len : 0; }
bool rtg_cache_is_empty(const rtg_cache* cache) { return rtg_cache_len(cache) == 0; }
void rtg_cache_clear(rtg_cache* cache) {
  if (cache) cache->len = 0;
}

void rtg_cache_destroy(rtg_cache* c) {
  if (!c) return;
  if (c->stream) hipStreamSynchronize(c->stream);
  destroy_graph(c);
  if (c->pstate) persistent_state_destroy(c->pstate);
  if (c->rstate) rows_state_destroy(c->rstate);
  free_work(c);
  for (void* p : {(void*)c->k, (void*)c->v, (void*)c->pos_dev, (void*)c->step_dev, (void*)c->keys,
                  (void*)c->token_dev, (void*)c->ids_dev, (void*)c->ids_in, (void*)c->logits,
                  (void*)c->bg_part, (void*)c->bg_cnt, (void*)c->bg_spart, (void*)c->bg_cen})
    if (p) hipFree(p);
  for (auto e : c->ev)
    if (e) hipEventDestroy(e);
  if (c->stream) hipStreamDestroy(c->stream);
  delete c;
}

rtg_result rtg_cache_read(const rtg_cache* c, size_t layer, size_t head, size_t seq, int values, float* out) {
  if (!c || !out) return err("null argument");
  const rtg_model* m = c->m;
  if (layer >= m->cfg.n_layer || head >= m->cfg.n_head || seq >= c->batch) return err("index out of range");
  const size_t P = m->cfg.n_positions, hd = m->hd;
  const float* base = (values ? c->v : c->k) + layer * c->layer_stride + ((seq * m->cfg.n_head + head) * P) * hd;
  try {
    if (c->len) HIPX(hipMemcpy(out, base, c->len * hd * 4, hipMemcpyDeviceToHost));
  } catch (const HipError& e) {
    return err(e.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_forward_cached_batched(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                                      float* logits_out) {
  if (!model || !cache) return err("null argument");
  if (cache->m != model) return err("the cache belongs to another model");
  std::string e = check_cached(model, cache->len, ids, n);
  if (e.empty() && cache->batch > 1) e = check_ids(model, ids, n * cache->batch);
  if (!e.empty()) return err(e);
  try {
    forward_cached_impl(cache, ids, n, logits_out);
  } catch (const HipError& he) {
    return err(he.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_forward_cached(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                              float* logits_out) {
  if (cache && cache->batch != 1) return err("rtg_forward_cached needs a batch-1 cache");
  return rtg_forward_cached_batched(model, cache, ids, n, logits_out);
}

// rtg_forward_cached_noalloc for a prompt the multi-row forward takes: its
// state in the scratch array (the 64 KiB head, then its work rows), the
// logits after it; the same kernel and inputs as rtg_forward_cached's.
static rtg_result noalloc_rows(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                               float* logits_out) {
  const size_t V = model->cfg.vocab_size;
  const size_t state = align_up(rows_state_bytes(model->rplan, false), 256) / 4;
  if (state + n * V > kScratchHeadFloats + kScratchFloats)
    return err(fmt("rtg_forward_cached_noalloc: %zu new tokens need %zu bytes of scratch; it holds %zu", n,
                   (state + n * V - kScratchHeadFloats) * 4, kScratchFloats * 4));
  try {
    hipError_t he = hipSuccess;
    float* sp = scratch_device_ptr(model->device, &he);
    HIPX(he);
    static_assert(rows_state_head_bytes() == kScratchHeadFloats * sizeof(float), "scratch head");
    std::lock_guard<std::mutex> slock(scratch_lock(model->device));
    std::lock_guard<std::mutex> plock(persistent_launch_lock(model->device));
    RowsState st;  // over the scratch array (one region per buffer): nothing is allocated
    st.mem = sp;
    st.fresh = false;
    float* logits = sp + state;
    HIPX(hipMemcpyAsync(cache->ids_in, ids, n * 4, hipMemcpyHostToDevice, cache->stream));
    enqueue_rows(cache, cache->ids_in, 1, n, cache->len, logits, &st);
    if (logits_out) HIPX(hipMemcpyAsync(logits_out, logits, n * V * 4, hipMemcpyDeviceToHost, cache->stream));
    HIPX(hipStreamSynchronize(cache->stream));
    check_rows(&st);
    cache->len += n;
  } catch (const HipError& he) {
    return err(he.msg);
  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_forward_cached_noalloc(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                                      float* logits_out) {
  if (!model || !cache || (n && !ids)) return err("null argument");
  // the pass runs cache->m's kernels on buffers sized from model's shape
  if (cache->m != model) return err("rtg_forward_cached_noalloc: the cache belongs to another model");
  if (cache->batch != 1) return err("rtg_forward_cached_noalloc needs a batch-1 cache");
  std::string e = check_cached(model, cache->len, ids, n);
  if (!e.empty()) return err(e);
  // x, ln, att [n][d], qkv [n][3d], h [n][4d], logits [n][V] in the device's
  // scratch array, each part on a 256-byte boundary like a hipMalloc'd buffer
  // (the same alignment, so the same kernels as rtg_forward_cached run)
  const size_t d = model->cfg.n_embd, V = model->cfg.vocab_size;
  const size_t pd = align_up(n * d, 64), p3 = align_up(3 * n * d, 64), p4 = align_up(4 * n * d, 64);
  const size_t pv = align_up(n * V, 64);
  // the split-k partial tiles the pass's GEMMs use at n rows (as much as the
  // cache's own workspace would hold for them, so the same kernels run)
  size_t pw = 0;
  for (const auto& nk : {std::make_pair(3 * d, d), std::make_pair(d, d), std::make_pair(4 * d, d),
                         std::make_pair(d, 4 * d)})
    pw = std::max(pw, gemm_splitk_ws_floats((int)n, (int)nk.first, (int)nk.second));
  pw = align_up(pw, 64);
  const size_t need = 3 * pd + p3 + p4 + pv;
  if (need > kScratchFloats)
    return err(fmt("rtg_forward_cached_noalloc: %zu new tokens need %zu bytes of scratch; it holds %zu", n,
                   need * 4, kScratchFloats * 4));
  // where the GEMMs' split-k partials do not fit beside the activations the
  // GEMMs run unsplit (the same sums in another order), so the limit is
  // exactly the activations' size and grows monotonically with n
  if (need + pw > kScratchFloats) pw = 0;
  if (rows_path(cache, 1, n)) return noalloc_rows(model, cache, ids, n, logits_out);
  try {
    hipError_t he = hipSuccess;
    float* sp = scratch_device_ptr(model->device, &he);
    HIPX(he);
    sp += kScratchHeadFloats;
    // every call on this device shares the array: one pass at a time (the
    // call has drained its stream when it returns)
    std::lock_guard<std::mutex> slock(scratch_lock(model->device));
    // Nothing here has to start at zero: every kernel of the pass writes its
    // output rows in full before they are read (the residual epilogues add
    // into x after the embedding has written it).
    Work w;
    w.x = sp;
    w.ln = w.x + pd;
    w.att = w.ln + pd;
    w.qkv = w.att + pd;
    w.h = w.qkv + p3;
    w.logits = w.h + p4;
    w.ws = pw ? w.logits + pv : nullptr;
    w.ws_floats = pw;
    HIPX(hipMemcpyAsync(cache->ids_in, ids, n * 4, hipMemcpyHostToDevice, cache->stream));
    enqueue_prefill(cache, w, cache->ids_in, 1, n, cache->len, 0);
    HIPX(hipGetLastError());
    if (logits_out)
      HIPX(hipMemcpyAsync(logits_out, w.logits, n * V * 4, hipMemcpyDeviceToHost, cache->stream));
    HIPX(hipStreamSynchronize(cache->stream));
    cache->len += n;
  } catch (const HipError& he) {
    return err(he.msg);
  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_forward(const rtg_model* model, const uint32_t* ids, size_t n, float* logits_out) {
  if (!model) return err("null argument");
  // gpt2.rs:269-279
  if (n == 0) return err("Empty input");
  if (n > model->cfg.n_positions)
    return err(fmt("Sequence length %zu exceeds max position %zu", n, model->cfg.n_positions));
  std::string e = check_ids(model, ids, n);
  if (!e.empty()) return err(e);
  try {
    PoolLease lease(model, 1);
    forward_cached_impl(lease.c, ids, n, logits_out);
  } catch (const HipError& he) {
    return err(he.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_generate_cached_batched(const rtg_model* model, const uint32_t* prompts, size_t batch, size_t n,
                                       size_t max_new, uint32_t* out, rtg_timing* timing) {
  if (!model || !out) return err("null argument");
  if (batch == 0) return err("batch must be >= 1");
  const size_t P = model->cfg.n_positions;
  std::string e = check_cached(model, 0, prompts, n);
  if (e.empty() && batch > 1) e = check_ids(model, prompts, n * batch);
  if (!e.empty()) return err(e);
  // The reference fails at the first decode step whose total exceeds
  // n_positions and discards the partial result (gpt2.rs:369-374, 427-433).
  const size_t steps = max_new > 0 ? max_new : 1;
  if (n + steps - 1 > P) return err(fmt("Total sequence length %zu exceeds max position %zu", P + 1, P));
  try {
    generate_greedy(model, prompts, batch, n, max_new, out, timing);
  } catch (const HipError& he) {
    return err(he.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_generate_cached(const rtg_model* model, const uint32_t* prompt, size_t n, size_t max_new,
                               float temperature, uint64_t seed, uint32_t* out) {
  if (temperature <= 0.0f) return rtg_generate_cached_batched(model, prompt, 1, n, max_new, out, nullptr);
  if (!model || !out) return err("null argument");
  // Sampling path (gpt2.rs:405-441 with sample_with_temperature, :996-1017),
  // tokens chosen on the device.
  std::string e = check_cached(model, 0, prompt, n);
  if (!e.empty()) return err(e);
  const size_t P = model->cfg.n_positions;
  const size_t steps = max_new > 0 ? max_new : 1;
  if (n + steps - 1 > P) return err(fmt("Total sequence length %zu exceeds max position %zu", P + 1, P));
  const SampleParams sp{temperature, 0, 1.0f, 1.0f, seed, 0};
  try {
    generate_greedy(model, prompt, 1, n, max_new, out, nullptr, &sp);
  } catch (const HipError& he) {
    return err(he.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_generate_with_config(const rtg_model* model, const uint32_t* prompt, size_t n,
                                    const rtg_gen_config* cfg, uint32_t* out) {
  if (!model || !out || !cfg) return err("null argument");
  if (cfg->temperature <= 0.0f && cfg->repetition_penalty == 1.0f)
    return rtg_generate_cached_batched(model, prompt, 1, n, cfg->max_new_tokens, out, nullptr);
  std::string e = check_cached(model, 0, prompt, n);
  if (!e.empty()) return err(e);
  const size_t P = model->cfg.n_positions;
  const size_t steps = cfg->max_new_tokens > 0 ? cfg->max_new_tokens : 1;
  if (n + steps - 1 > P) return err(fmt("Total sequence length %zu exceeds max position %zu", P + 1, P));
  // sample_logits (gpt2.rs:871-906) on the device after every step
  const int k = cfg->top_k > (size_t)INT32_MAX ? INT32_MAX : (int)cfg->top_k;
  const SampleParams sp{cfg->temperature, k, cfg->top_p, cfg->repetition_penalty, cfg->seed, 0};
  try {
    generate_greedy(model, prompt, 1, n, cfg->max_new_tokens, out, nullptr, &sp);
  } catch (const HipError& he) {
    return err(he.msg);  } catch (const std::exception& ex) {
    return err_internal(ex);
  }
  return ok();
}

rtg_result rtg_generate(const rtg_model* model, const uint32_t* prompt, size_t n, size_t max_new, float temperature,
                        uint64_t seed, uint32_t* out) {
  if (!model || !out) return err("null argument");
  // gpt2.rs:311-346: each step runs forward() over the last n_positions
  // tokens and picks the next token from the last row's logits. The tokens
  // live in one device buffer: the step reads its window from there and the
  // device sampler appends its choice, so the loop never waits for the host.
  const size_t V = model->cfg.vocab_size, P = model->cfg.n_positions;
  if (max_new == 0) {
    memcpy(out, prompt, n * 4);
    return ok();
  }
  if (n == 0) return err("Empty input");
  // forward() checks the ids of each window; later windows add only sampled ids
  const size_t start0 = n > P ? n - P : 0;
  std::string e = check_ids(model, prompt + start0, n - start0);
  if (!e.empty()) return err(e);
  const size_t total = n + max_new;
  uint32_t* toks = nullptr;
  int* steps = nullptr;
  try {
    PoolLease lease(model, 1);
    rtg_cache* c = lease.c;
    hipStream_t s = c->stream;
    HIPX(hipMalloc(&toks, total * 4));
    HIPX(hipMalloc(&steps, max_new * 4));
    std::vector<int> step_no(max_new);
    for (size_t i = 0; i < max_new; ++i) step_no[i] = (int)(i + 1);  // the sampler's generation index + 1
    HIPX(hipMemcpyAsync(toks, prompt, n * 4, hipMemcpyHostToDevice, s));
    HIPX(hipMemcpyAsync(steps, step_no.data(), max_new * 4, hipMemcpyHostToDevice, s));
    c->len = 0;
    ensure_rows(c, std::min(total - 1, P));
    ensure_logits(c, 1);
    // sample_with_temperature (gpt2.rs:996-1017); argmax for temperature <= 0.
    // Draw k of the seeded sequence goes to generation index k - 1.
    const SampleParams sp{temperature, 0, 1.0f, 1.0f, seed, 0};
    for (size_t i = 0; i < max_new; ++i) {
      const size_t len = n + i;
      const size_t start = len > P ? len - P : 0;
      enqueue_prefill(c, cache_work(c), toks + start, 1, len - start, 0, 1);  // logits of the last row only
      if (!launch_sample(s, c->logits, (int)V, toks, (int)n, toks + n, steps + i, sp, c->token_dev))
        throw HipError{"vocabulary too large for the device sampler"};
    }
    HIPX(hipMemcpyAsync(out, toks, total * 4, hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    c->len = 0;
  } catch (const HipError& he) {
    if (toks) hipFree(toks);
    if (steps) hipFree(steps);
    return err(he.msg);  } catch (const std::exception& ex) {
    if (toks) hipFree(toks);
    if (steps) hipFree(steps);
    return err_internal(ex);
  }
  hipFree(toks);
  hipFree(steps);
  return ok();
}

}  // extern "C"
