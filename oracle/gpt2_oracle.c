/* CPU oracle for the GPT-2 token loop (test infrastructure only; see
 * gpt2_oracle.h). Plain-C restatement of rusttorch-core/src/nn/gpt2.rs.
 *
 * Parity pins (each checked by tests/test_oracle.py):
 *  - embedding_lookup, slice_columns, argmax, KV append/clear: exact closed
 *    forms and the reference's own unit tests (gpt2.rs:1174-1238, 1456-1503).
 *  - layer_norm, gelu_new, attention, matmul: float64 closed forms, brute force
 *    on tiny inputs, the reference's known values (gpt2.rs:1192-1222, 1280-1291).
 *  - whole forward / greedy loop: a locally constructed transformers
 *    GPT2LMHeadModel on identical weights, a float64 numpy restatement, and the
 *    reference's self-consistency tests (cached == uncached == incremental,
 *    gpt2.rs:1506-1602).
 * Summation order of the reference's sgemm (ndarray 0.15 -> matrixmultiply
 * 0.3, not vendored) is "parity unpinned": only value-level agreement within
 * tolerance is claimed for matmul-derived results. */
#include "gpt2_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct orc_layer {
  const float *ln_1_w, *ln_1_b, *c_attn_w, *c_attn_b, *c_proj_w, *c_proj_b;
  const float *ln_2_w, *ln_2_b, *fc_w, *fc_b, *mproj_w, *mproj_b;
};

struct orc_model {
  orc_config cfg;
  const float *wte, *wpe, *ln_f_w, *ln_f_b;
  struct orc_layer* layers;
  int threads;
  int lm_direct; /* lm_head without the materialised transpose (same values) */
};

/* KVCache / LayerKVCache (gpt2.rs:111-175): keys[layer][head] hold
 * cached_len * head_dim floats; storage is preallocated for n_positions, which
 * behaves like the reference's growable Vec for every reachable length. */
struct orc_cache {
  size_t n_layer, n_head, head_dim, cap;
  size_t* cached_len; /* per layer */
  float* keys;        /* [layer][head][cap][head_dim] */
  float* values;
};

/* ---- helpers (gpt2.rs:605-868) ---- */

/* embedding_lookup, gpt2.rs:607-625. */
int orc_embedding_lookup(const float* weight, size_t rows, size_t n_embd, const uint32_t* ids, size_t n,
                         float* out, char* err) {
  for (size_t i = 0; i < n; ++i) {
    size_t idx = ids[i];
    if (idx >= rows) {
      if (err) snprintf(err, 256, "Token ID %zu out of range (vocab_size=%zu)", idx, rows);
      return -1;
    }
    memcpy(out + i * n_embd, weight + idx * n_embd, n_embd * sizeof(float));
  }
  return 0;
}

/* layer_norm, gpt2.rs:636-666: mean and variance are sequential f32 folds. */
void orc_layer_norm(const float* x, size_t rows, size_t n, const float* w, const float* b, float eps, float* out) {
  for (size_t i = 0; i < rows; ++i) {
    const float* row = x + i * n;
    float sum = 0.0f;
    for (size_t j = 0; j < n; ++j) sum += row[j];
    float mean = sum / (float)n;
    float vs = 0.0f;
    for (size_t j = 0; j < n; ++j) {
      float d = row[j] - mean;
      vs += d * d;
    }
    float var = vs / (float)n;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (size_t j = 0; j < n; ++j) out[i * n + j] = (row[j] - mean) * inv_std * w[j] + b[j];
  }
}

/* matrix::matmul (ops/matrix.rs:36-117) for 2D f32: out[m,n] = a[m,k] @ b[k,n].
 * Each output element starts from 0.0f and adds a[i][kk] * b[kk][j] for kk in
 * ascending order (one rounded product, one rounded add per term). The tiles
 * below only decide which elements are accumulated together (in registers,
 * MI x NJ at a time); no element's order depends on the tiling or on the
 * thread count. */
enum { MI = 4, NJ = 32, MROWS = 64 };

/* rows [i0, i0 + ni) (ni <= MI) x columns [j0, j0 + NJ) */
static void mm_tile(const float* a, size_t k, const float* b, size_t n, float* out, size_t i0, size_t ni, size_t j0) {
  float acc[MI][NJ];
  memset(acc, 0, sizeof acc);
  if (ni == MI) {
    for (size_t kk = 0; kk < k; ++kk) {
      const float* br = b + kk * n + j0;
      const float a0 = a[(i0 + 0) * k + kk], a1 = a[(i0 + 1) * k + kk];
      const float a2 = a[(i0 + 2) * k + kk], a3 = a[(i0 + 3) * k + kk];
      for (int j = 0; j < NJ; ++j) {
        acc[0][j] += a0 * br[j];
        acc[1][j] += a1 * br[j];
        acc[2][j] += a2 * br[j];
        acc[3][j] += a3 * br[j];
      }
    }
  } else {
    for (size_t ii = 0; ii < ni; ++ii)
      for (size_t kk = 0; kk < k; ++kk) {
        const float* br = b + kk * n + j0;
        const float av = a[(i0 + ii) * k + kk];
        for (int j = 0; j < NJ; ++j) acc[ii][j] += av * br[j];
      }
  }
  for (size_t ii = 0; ii < ni; ++ii) memcpy(out + (i0 + ii) * n + j0, acc[ii], NJ * sizeof(float));
}

void orc_matmul(const float* a, size_t m, size_t k, const float* b, size_t n, float* out, int threads) {
  const long njb = (long)(n / NJ), nmb = (long)((m + MROWS - 1) / MROWS);
  (void)threads;
  /* full column blocks: work items (row group, column block) */
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads > 0 ? threads : 1) if (threads > 1)
  for (long w = 0; w < njb * nmb; ++w) {
    const size_t j0 = (size_t)(w % njb) * NJ, r0 = (size_t)(w / njb) * MROWS;
    const size_t r1 = r0 + MROWS < m ? r0 + MROWS : m;
    for (size_t i0 = r0; i0 < r1; i0 += MI) mm_tile(a, k, b, n, out, i0, r1 - i0 < MI ? r1 - i0 : MI, j0);
  }
  /* the last n % NJ columns */
  const size_t jt = (size_t)njb * NJ;
  if (jt < n)
    for (size_t i = 0; i < m; ++i)
      for (size_t j = jt; j < n; ++j) {
        float acc = 0.0f;
        for (size_t kk = 0; kk < k; ++kk) acc += a[i * k + kk] * b[kk * n + j];
        out[i * n + j] = acc;
      }
}

/* conv1d_forward, gpt2.rs:628-633: y = x @ W + b, W is [in, out]; the bias
 * add is broadcast::add_broadcast (broadcast.rs:177-180) = plain f32 add. */
void orc_conv1d(const float* x, size_t rows, size_t k, const float* w, const float* bias, size_t n, float* out,
                int threads) {
  orc_matmul(x, rows, k, w, n, out, threads);
  for (size_t i = 0; i < rows; ++i)
    for (size_t j = 0; j < n; ++j) out[i * n + j] = out[i * n + j] + bias[j];
}

/* slice_columns, gpt2.rs:669-683. */
void orc_slice_columns(const float* t, size_t rows, size_t cols, size_t start, size_t end, float* out) {
  size_t oc = end - start;
  for (size_t i = 0; i < rows; ++i)
    for (size_t j = 0; j < oc; ++j) out[i * oc + j] = t[i * cols + start + j];
}

/* Softmax as written in gpt2.rs:805-817 and 724-737: max by an f32::max fold
 * from -inf (fmaxf ignores NaN like f32::max), exp(s - max), sequential sum,
 * then divide each entry. */
static void softmax_inplace(float* s, size_t n) {
  float mx = -INFINITY;
  for (size_t j = 0; j < n; ++j) mx = fmaxf(mx, s[j]);
  float sum = 0.0f;
  for (size_t j = 0; j < n; ++j) {
    s[j] = expf(s[j] - mx);
    sum += s[j];
  }
  for (size_t j = 0; j < n; ++j) s[j] /= sum;
}

/* multi_head_attention (uncached, causal), gpt2.rs:686-750. */
void orc_multi_head_attention(const float* q, const float* k, const float* v, size_t n_head, size_t head_dim,
                              size_t seq_len, float* out) {
  size_t n_embd = n_head * head_dim;
  float scale = 1.0f / sqrtf((float)head_dim);
  float* scores = (float*)malloc(seq_len * seq_len * sizeof(float));
  for (size_t h = 0; h < n_head; ++h) {
    size_t off = h * head_dim;
    for (size_t i = 0; i < seq_len; ++i) {
      for (size_t j = 0; j < seq_len; ++j) {
        if (j > i) {
          scores[i * seq_len + j] = -INFINITY;
        } else {
          float dot = 0.0f;
          for (size_t d = 0; d < head_dim; ++d) dot += q[i * n_embd + off + d] * k[j * n_embd + off + d];
          scores[i * seq_len + j] = dot * scale;
        }
      }
    }
    for (size_t i = 0; i < seq_len; ++i) softmax_inplace(scores + i * seq_len, seq_len);
    for (size_t i = 0; i < seq_len; ++i) {
      for (size_t d = 0; d < head_dim; ++d) {
        float val = 0.0f;
        for (size_t j = 0; j < seq_len; ++j) val += scores[i * seq_len + j] * v[j * n_embd + off + d];
        out[i * n_embd + off + d] = val;
      }
    }
  }
  free(scores);
}

/* gelu_new, gpt2.rs:837-847. sqrt(2/pi) is computed in f32 as the reference
 * does: (2.0f32 / PI).sqrt(). */
void orc_gelu_new(const float* x, size_t n, float* out) {
  const float sqrt_2_pi = sqrtf(2.0f / (float)3.14159265358979323846);
  for (size_t i = 0; i < n; ++i) {
    float xv = x[i];
    float inner = sqrt_2_pi * (xv + 0.044715f * xv * xv * xv);
    out[i] = 0.5f * xv * (1.0f + tanhf(inner));
  }
}

/* argmax_f32, gpt2.rs:858-868: strict '>' scan from -inf; first maximum
 * wins, NaN never wins, an all-NaN (or all -inf) row gives 0. */
uint32_t orc_argmax(const float* data, size_t n) {
  size_t best = 0;
  float bv = -INFINITY;
  for (size_t i = 0; i < n; ++i) {
    if (data[i] > bv) {
      bv = data[i];
      best = i;
    }
  }
  return (uint32_t)best;
}

/* apply_repetition_penalty, gpt2.rs:910-921. */
void orc_apply_repetition_penalty(float* logits, size_t n, const uint32_t* tokens, size_t nt, float penalty) {
  for (size_t t = 0; t < nt; ++t) {
    size_t idx = tokens[t];
    if (idx < n) {
      if (logits[idx] > 0.0f)
        logits[idx] /= penalty;
      else
        logits[idx] *= penalty;
    }
  }
}

static int cmp_desc(const void* pa, const void* pb) {
  float a = *(const float*)pa, b = *(const float*)pb;
  if (a > b) return -1;
  if (a < b) return 1;
  return 0;
}

/* apply_top_k, gpt2.rs:924-935: threshold = k-th largest, strictly smaller
 * entries become -inf (ties at the threshold are all kept). */
void orc_apply_top_k(float* logits, size_t n, size_t k) {
  if (n == 0 || k == 0) return;
  float* sorted = (float*)malloc(n * sizeof(float));
  memcpy(sorted, logits, n * sizeof(float));
  qsort(sorted, n, sizeof(float), cmp_desc);
  float thr = sorted[(k < n ? k : n) - 1];
  for (size_t i = 0; i < n; ++i)
    if (logits[i] < thr) logits[i] = -INFINITY;
  free(sorted);
}

static const float* g_sort_probs;
static int cmp_idx_desc(const void* pa, const void* pb) {
  size_t a = *(const size_t*)pa, b = *(const size_t*)pb;
  float fa = g_sort_probs[a], fb = g_sort_probs[b];
  if (fa > fb) return -1;
  if (fa < fb) return 1;
  return a < b ? -1 : (a > b ? 1 : 0); /* stable like Rust's sort_by */
}

/* apply_top_p, gpt2.rs:939-967: softmax, descending stable sort, keep tokens
 * until the running sum (f32) reaches p. */
void orc_apply_top_p(float* logits, size_t n, float p) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, logits[i]);
  float* probs = (float*)malloc(n * sizeof(float));
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    probs[i] = expf(logits[i] - mx);
    sum += probs[i];
  }
  for (size_t i = 0; i < n; ++i) probs[i] = probs[i] / sum;
  size_t* idx = (size_t*)malloc(n * sizeof(size_t));
  for (size_t i = 0; i < n; ++i) idx[i] = i;
  g_sort_probs = probs;
  qsort(idx, n, sizeof(size_t), cmp_idx_desc);
  unsigned char* keep = (unsigned char*)calloc(n, 1);
  float cum = 0.0f;
  for (size_t r = 0; r < n; ++r) {
    keep[idx[r]] = 1;
    cum += probs[idx[r]];
    if (cum >= p) break;
  }
  for (size_t i = 0; i < n; ++i)
    if (!keep[i]) logits[i] = -INFINITY;
  free(keep);
  free(idx);
  free(probs);
}

/* ---- model (gpt2.rs:214-263) ---- */

static const float* find_w(const char* const* names, const float* const* ptrs, size_t n, const char* want) {
  for (size_t i = 0; i < n; ++i)
    if (strcmp(names[i], want) == 0) return ptrs[i];
  return NULL;
}

int orc_model_create(const orc_config* cfg, const char* const* names, const float* const* ptrs, size_t n,
                     orc_model** out, char* err) {
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->cfg = *cfg;
  m->threads = 1;
  m->layers = (struct orc_layer*)calloc(cfg->n_layer ? cfg->n_layer : 1, sizeof(struct orc_layer));
  char nm[128];
#define GET(dst, ...)                                               \
  do {                                                              \
    snprintf(nm, sizeof nm, __VA_ARGS__);                           \
    (dst) = find_w(names, ptrs, n, nm);                             \
    if (!(dst)) {                                                   \
      if (err) snprintf(err, 256, "Missing weight: %s", nm);        \
      orc_model_destroy(m);                                         \
      return -1;                                                    \
    }                                                               \
  } while (0)
  GET(m->wte, "wte.weight");
  GET(m->wpe, "wpe.weight");
  GET(m->ln_f_w, "ln_f.weight");
  GET(m->ln_f_b, "ln_f.bias");
  for (size_t i = 0; i < cfg->n_layer; ++i) {
    struct orc_layer* L = &m->layers[i];
    GET(L->ln_1_w, "h.%zu.ln_1.weight", i);
    GET(L->ln_1_b, "h.%zu.ln_1.bias", i);
    GET(L->c_attn_w, "h.%zu.attn.c_attn.weight", i);
    GET(L->c_attn_b, "h.%zu.attn.c_attn.bias", i);
    GET(L->c_proj_w, "h.%zu.attn.c_proj.weight", i);
    GET(L->c_proj_b, "h.%zu.attn.c_proj.bias", i);
    GET(L->ln_2_w, "h.%zu.ln_2.weight", i);
    GET(L->ln_2_b, "h.%zu.ln_2.bias", i);
    GET(L->fc_w, "h.%zu.mlp.c_fc.weight", i);
    GET(L->fc_b, "h.%zu.mlp.c_fc.bias", i);
    GET(L->mproj_w, "h.%zu.mlp.c_proj.weight", i);
    GET(L->mproj_b, "h.%zu.mlp.c_proj.bias", i);
  }
#undef GET
  *out = m;
  return 0;
}

void orc_model_destroy(orc_model* m) {
  if (!m) return;
  free(m->layers);
  free(m);
}

void orc_model_set_threads(orc_model* m, int threads) { m->threads = threads > 0 ? threads : 1; }

void orc_model_set_lm_direct(orc_model* m, int on) { m->lm_direct = on != 0; }

/* num_parameters, gpt2.rs:541-563. */
size_t orc_num_parameters(const orc_model* m) {
  size_t d = m->cfg.n_embd, f = 4 * d;
  size_t per_layer = 2 * d + d * 3 * d + 3 * d + d * d + d + 2 * d + d * f + f + f * d + d;
  return m->cfg.vocab_size * d + m->cfg.n_positions * d + 2 * d + m->cfg.n_layer * per_layer;
}

orc_cache* orc_cache_new(const orc_model* m) {
  orc_cache* c = (orc_cache*)calloc(1, sizeof(orc_cache));
  c->n_layer = m->cfg.n_layer;
  c->n_head = m->cfg.n_head;
  c->head_dim = m->cfg.n_embd / m->cfg.n_head;
  c->cap = m->cfg.n_positions;
  c->cached_len = (size_t*)calloc(c->n_layer ? c->n_layer : 1, sizeof(size_t));
  size_t sz = c->n_layer * c->n_head * c->cap * c->head_dim;
  c->keys = (float*)calloc(sz ? sz : 1, sizeof(float));
  c->values = (float*)calloc(sz ? sz : 1, sizeof(float));
  return c;
}

/* KVCache::len, gpt2.rs:137-143: layer 0's cached_len. */
size_t orc_cache_len(const orc_cache* c) { return c->n_layer ? c->cached_len[0] : 0; }

void orc_cache_clear(orc_cache* c) {
  for (size_t l = 0; l < c->n_layer; ++l) c->cached_len[l] = 0;
}

void orc_cache_destroy(orc_cache* c) {
  if (!c) return;
  free(c->cached_len);
  free(c->keys);
  free(c->values);
  free(c);
}

static float* kv_ptr(const orc_cache* c, float* base, size_t l, size_t h) {
  return base + ((l * c->n_head + h) * c->cap) * c->head_dim;
}

int orc_cache_read(const orc_cache* c, size_t layer, size_t head, int values, float* out) {
  if (layer >= c->n_layer || head >= c->n_head) return -1;
  const float* src = kv_ptr(c, values ? c->values : c->keys, layer, head);
  memcpy(out, src, c->cached_len[layer] * c->head_dim * sizeof(float));
  return 0;
}

/* multi_head_attention_cached, gpt2.rs:772-834 over this layer's cache.
 * Every (head, row) pair is independent; with threads > 1 they are spread
 * over threads, each computing its pairs exactly as the single-threaded loop
 * does (scores in j order, softmax_inplace, then each output dim summed over
 * j in ascending order). */
static void attention_cached(const orc_cache* c, size_t layer, const float* q, size_t new_len, size_t past_len,
                             float* out, int threads) {
  size_t hd = c->head_dim, nh = c->n_head, n_embd = nh * hd;
  float scale = 1.0f / sqrtf((float)hd);
  const long rows = (long)(nh * new_len);
#pragma omp parallel num_threads(threads > 0 ? threads : 1) if (threads > 1 && rows > 1)
  {
    float* scores = (float*)malloc((past_len + new_len) * sizeof(float));
    float* val = (float*)malloc(hd * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (long r = 0; r < rows; ++r) {
      const size_t h = (size_t)r / new_len, i = new_len - 1 - (size_t)r % new_len; /* longest rows first */
      const float* K = kv_ptr(c, c->keys, layer, h);
      const float* V = kv_ptr(c, c->values, layer, h);
      size_t attend = past_len + i + 1;
      const float* qi = q + i * n_embd + h * hd;
      for (size_t j = 0; j < attend; ++j) {
        float dot = 0.0f;
        for (size_t d = 0; d < hd; ++d) dot += qi[d] * K[j * hd + d];
        scores[j] = dot * scale;
      }
      softmax_inplace(scores, attend);
      for (size_t d = 0; d < hd; ++d) val[d] = 0.0f;
      for (size_t j = 0; j < attend; ++j) {
        const float sj = scores[j];
        for (size_t d = 0; d < hd; ++d) val[d] += sj * V[j * hd + d];
      }
      for (size_t d = 0; d < hd; ++d) out[i * n_embd + h * hd + d] = val[d];
    }
    free(val);
    free(scores);
  }
}

static void vec_add(const float* a, const float* b, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* One pre-LN block; cache == NULL selects forward_layer (gpt2.rs:566-601),
 * otherwise forward_layer_cached (gpt2.rs:477-538). x is updated in place. */
static void run_layer(const orc_model* m, size_t li, float* x, size_t T, orc_cache* cache, size_t past_len) {
  const struct orc_layer* L = &m->layers[li];
  size_t d = m->cfg.n_embd, nh = m->cfg.n_head, hd = d / nh, f = 4 * d;
  float eps = m->cfg.layer_norm_epsilon;
  int th = m->threads;
  float* ln = (float*)malloc(T * d * sizeof(float));
  float* qkv = (float*)malloc(T * 3 * d * sizeof(float));
  float* q = (float*)malloc(T * d * sizeof(float));
  float* k = (float*)malloc(T * d * sizeof(float));
  float* v = (float*)malloc(T * d * sizeof(float));
  float* att = (float*)malloc(T * d * sizeof(float));
  float* proj = (float*)malloc(T * d * sizeof(float));
  float* fc = (float*)malloc(T * f * sizeof(float));
  float* act = (float*)malloc(T * f * sizeof(float));

  /* row-wise ops (LayerNorm, gelu_new) split over rows when threaded: each
   * row is computed exactly as the single-threaded call computes it */
#pragma omp parallel for num_threads(th) if (th > 1 && T > 1)
  for (long i = 0; i < (long)T; ++i) orc_layer_norm(x + i * d, 1, d, L->ln_1_w, L->ln_1_b, eps, ln + i * d);
  orc_conv1d(ln, T, d, L->c_attn_w, L->c_attn_b, 3 * d, qkv, th);
  orc_slice_columns(qkv, T, 3 * d, 0, d, q);
  orc_slice_columns(qkv, T, 3 * d, d, 2 * d, k);
  orc_slice_columns(qkv, T, 3 * d, 2 * d, 3 * d, v);
  if (cache) {
    /* LayerKVCache::append with the per-head split of gpt2.rs:500-514. */
    for (size_t pos = 0; pos < T; ++pos)
      for (size_t h = 0; h < nh; ++h) {
        memcpy(kv_ptr(cache, cache->keys, li, h) + (past_len + pos) * hd, k + pos * d + h * hd, hd * sizeof(float));
        memcpy(kv_ptr(cache, cache->values, li, h) + (past_len + pos) * hd, v + pos * d + h * hd,
               hd * sizeof(float));
      }
    cache->cached_len[li] += T;
    attention_cached(cache, li, q, T, past_len, att, th);
  } else {
    orc_multi_head_attention(q, k, v, nh, hd, T, att);
  }
  orc_conv1d(att, T, d, L->c_proj_w, L->c_proj_b, d, proj, th);
  vec_add(x, proj, x, T * d); /* x2 = x + attn_proj */
#pragma omp parallel for num_threads(th) if (th > 1 && T > 1)
  for (long i = 0; i < (long)T; ++i) orc_layer_norm(x + i * d, 1, d, L->ln_2_w, L->ln_2_b, eps, ln + i * d);
  orc_conv1d(ln, T, d, L->fc_w, L->fc_b, f, fc, th);
#pragma omp parallel for num_threads(th) if (th > 1 && T > 1)
  for (long i = 0; i < (long)T; ++i) orc_gelu_new(fc + i * f, f, act + i * f);
  orc_conv1d(act, T, f, L->mproj_w, L->mproj_b, d, proj, th);
  vec_add(x, proj, x, T * d); /* x2 + proj */

  free(ln); free(qkv); free(q); free(k); free(v); free(att); free(proj); free(fc); free(act);
}

/* Shared tail: ln_f then the tied LM head x @ wte^T (gpt2.rs:392-396). The
 * transpose is materialised as matrix::transpose does (the reference's cost
 * per call), unless lm_direct is set: then each logit is summed straight from
 * the contiguous wte row, over j in ascending order from 0.0f, which is the
 * same arithmetic as the matmul over the transposed copy (bit-identical). */
static void lm_head(const orc_model* m, const float* x, size_t T, float* logits) {
  size_t d = m->cfg.n_embd, V = m->cfg.vocab_size;
  float* ln = (float*)malloc(T * d * sizeof(float));
  orc_layer_norm(x, T, d, m->ln_f_w, m->ln_f_b, m->cfg.layer_norm_epsilon, ln);
  if (m->lm_direct && T <= 8) { /* (many rows: the tiled matmul is faster) */
#pragma omp parallel for schedule(static) num_threads(m->threads > 0 ? m->threads : 1) if (m->threads > 1)
    for (long v = 0; v < (long)V; ++v) {
      const float* w = m->wte + (size_t)v * d;
      for (size_t i = 0; i < T; ++i) {
        float acc = 0.0f;
        for (size_t j = 0; j < d; ++j) acc += ln[i * d + j] * w[j];
        logits[i * V + (size_t)v] = acc;
      }
    }
    free(ln);
    return;
  }
  float* wt = (float*)malloc(d * V * sizeof(float));
  /* the same copy, in 64 x 64 blocks so that reads and writes stay in cache */
  const long nvb = (long)((V + 63) / 64);
#pragma omp parallel for schedule(static) num_threads(m->threads > 0 ? m->threads : 1) if (m->threads > 1)
  for (long vb = 0; vb < nvb; ++vb)
    for (size_t j0 = 0; j0 < d; j0 += 64)
      for (size_t v = (size_t)vb * 64; v < V && v < (size_t)vb * 64 + 64; ++v)
        for (size_t j = j0; j < d && j < j0 + 64; ++j) wt[j * V + v] = m->wte[v * d + j];
  orc_matmul(ln, T, d, wt, V, logits, m->threads);
  free(wt);
  free(ln);
}

static int embed(const orc_model* m, const uint32_t* ids, size_t T, size_t pos0, float* x, char* err) {
  size_t d = m->cfg.n_embd;
  float* pe = (float*)malloc(T * d * sizeof(float));
  if (orc_embedding_lookup(m->wte, m->cfg.vocab_size, d, ids, T, x, err) != 0) {
    free(pe);
    return -1;
  }
  for (size_t i = 0; i < T; ++i) memcpy(pe + i * d, m->wpe + (pos0 + i) * d, d * sizeof(float));
  vec_add(x, pe, x, T * d);
  free(pe);
  return 0;
}

/* forward, gpt2.rs:269-304. */
int orc_forward(const orc_model* m, const uint32_t* ids, size_t n, float* logits, char* err) {
  if (n == 0) {
    if (err) snprintf(err, 256, "Empty input");
    return -1;
  }
  if (n > m->cfg.n_positions) {
    if (err) snprintf(err, 256, "Sequence length %zu exceeds max position %zu", n, m->cfg.n_positions);
    return -1;
  }
  float* x = (float*)malloc(n * m->cfg.n_embd * sizeof(float));
  if (embed(m, ids, n, 0, x, err) != 0) {
    free(x);
    return -1;
  }
  for (size_t l = 0; l < m->cfg.n_layer; ++l) run_layer(m, l, x, n, NULL, 0);
  lm_head(m, x, n, logits);
  free(x);
  return 0;
}

/* forward_cached, gpt2.rs:358-399. Error order: empty, overlength, token id;
 * the cache is untouched on every error. */
int orc_forward_cached(const orc_model* m, orc_cache* c, const uint32_t* ids, size_t n, float* logits, char* err) {
  if (n == 0) {
    if (err) snprintf(err, 256, "Empty input");
    return -1;
  }
  size_t past = orc_cache_len(c), total = past + n;
  if (total > m->cfg.n_positions) {
    if (err) snprintf(err, 256, "Total sequence length %zu exceeds max position %zu", total, m->cfg.n_positions);
    return -1;
  }
  float* x = (float*)malloc(n * m->cfg.n_embd * sizeof(float));
  if (embed(m, ids, n, past, x, err) != 0) {
    free(x);
    return -1;
  }
  for (size_t l = 0; l < m->cfg.n_layer; ++l) run_layer(m, l, x, n, c, past);
  lm_head(m, x, n, logits);
  free(x);
  return 0;
}

/* generate_cached with temperature <= 0, gpt2.rs:405-441. The prefill token
 * is pushed even when max_new == 0, as in the reference. */
/* Top-1 minus top-2 value of a logits row (NaN skipped; a tie at the top gives
 * 0): the margin by which the greedy choice of that row won. Diagnostic only,
 * for telling a near tie from a wrong logit when greedy ids differ. */
float orc_top2_gap(const float* data, size_t n) {
  float b1 = -INFINITY, b2 = -INFINITY;
  for (size_t i = 0; i < n; ++i) {
    const float v = data[i];
    if (v > b1) {
      b2 = b1;
      b1 = v;
    } else if (v > b2) {
      b2 = v;
    }
  }
  return (b1 > -INFINITY && b2 > -INFINITY) ? b1 - b2 : INFINITY;
}

int orc_generate_cached(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out,
                        char* err) {
  return orc_generate_cached_gaps(m, prompt, n, max_new, out, NULL, err);
}

int orc_generate_cached_gaps(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out,
                             float* gaps, char* err) {
  size_t V = m->cfg.vocab_size;
  orc_cache* c = orc_cache_new(m);
  float* logits = (float*)malloc((n ? n : 1) * V * sizeof(float));
  int rc = orc_forward_cached(m, c, prompt, n, logits, err);
  if (rc == 0) {
    memcpy(out, prompt, n * sizeof(uint32_t));
    size_t len = n;
    out[len++] = orc_argmax(logits + (n - 1) * V, V);
    if (gaps) gaps[0] = orc_top2_gap(logits + (n - 1) * V, V);
    for (size_t s = 1; s < max_new; ++s) {
      uint32_t last = out[len - 1];
      rc = orc_forward_cached(m, c, &last, 1, logits, err);
      if (rc != 0) break;
      if (gaps) gaps[s] = orc_top2_gap(logits, V);
      out[len++] = orc_argmax(logits, V);
    }
  }
  free(logits);
  orc_cache_destroy(c);
  return rc;
}

/* generate (uncached) with temperature <= 0, gpt2.rs:311-346: each step runs
 * forward over the last n_positions tokens (sliding window). */
int orc_generate(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out, char* err) {
  size_t V = m->cfg.vocab_size, P = m->cfg.n_positions;
  memcpy(out, prompt, n * sizeof(uint32_t));
  size_t len = n;
  size_t win_max = (n + max_new) < P ? (n + max_new) : P;
  float* logits = (float*)malloc((win_max ? win_max : 1) * V * sizeof(float));
  int rc = 0;
  for (size_t s = 0; s < max_new; ++s) {
    size_t start = len > P ? len - P : 0;
    size_t ctx = len - start;
    rc = orc_forward(m, out + start, ctx, logits, err);
    if (rc != 0) break;
    out[len++] = orc_argmax(logits + (ctx - 1) * V, V);
  }
  free(logits);
  return rc;
}
