/* CPU oracle for the GPT-2 token loop: a plain-C restatement of
 * rusttorch-core/src/nn/gpt2.rs (reference, read as text).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * the timed CPU baseline. The product library (librtgpu.so) never links,
 * loads or calls it.
 *
 * Every routine keeps the reference's operation order: sequential f32 folds,
 * no fused multiply-add (built with -ffp-contract=off), glibc expf/tanhf/sqrtf.
 * The one documented departure is matmul: the reference calls ndarray's dot
 * (matrixmultiply sgemm, an external crate whose blocking and summation order
 * are not pinned by anything in the reference); this oracle sums each output
 * element over k in ascending order. */
#ifndef RUSTTORCH_GPT2_ORACLE_H
#define RUSTTORCH_GPT2_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
  size_t vocab_size, n_positions, n_embd, n_layer, n_head;
  float layer_norm_epsilon;
} orc_config;

typedef struct orc_model orc_model;
typedef struct orc_cache orc_cache;

/* Helpers, each following one function of gpt2.rs. Return 0 on success, or
 * -1 and fill err (>= 256 bytes) with the reference's message. */
int orc_embedding_lookup(const float* weight, size_t rows, size_t n_embd, const uint32_t* ids, size_t n,
                         float* out, char* err);
void orc_layer_norm(const float* x, size_t rows, size_t n, const float* w, const float* b, float eps, float* out);
void orc_conv1d(const float* x, size_t rows, size_t k, const float* w, const float* bias, size_t n, float* out,
                int threads);
void orc_matmul(const float* a, size_t m, size_t k, const float* b, size_t n, float* out, int threads);
void orc_slice_columns(const float* t, size_t rows, size_t cols, size_t start, size_t end, float* out);
void orc_multi_head_attention(const float* q, const float* k, const float* v, size_t n_head, size_t head_dim,
                              size_t seq_len, float* out);
void orc_gelu_new(const float* x, size_t n, float* out);
uint32_t orc_argmax(const float* data, size_t n);
void orc_apply_repetition_penalty(float* logits, size_t n, const uint32_t* tokens, size_t nt, float penalty);
void orc_apply_top_k(float* logits, size_t n, size_t k);
void orc_apply_top_p(float* logits, size_t n, float p);

/* Model: from_state_dict over (name, pointer) pairs. Pointers are borrowed. */
int orc_model_create(const orc_config* cfg, const char* const* names, const float* const* ptrs, size_t n,
                     orc_model** out, char* err);
void orc_model_destroy(orc_model* m);
void orc_model_set_threads(orc_model* m, int threads);
/* on != 0: the tied LM head sums each logit from its wte row instead of
 * multiplying by a materialised transpose (the reference's per-call copy,
 * gpt2.rs:395). Same arithmetic per logit, so the same values; faster. */
void orc_model_set_lm_direct(orc_model* m, int on);
size_t orc_num_parameters(const orc_model* m);

orc_cache* orc_cache_new(const orc_model* m);
size_t orc_cache_len(const orc_cache* c);
void orc_cache_clear(orc_cache* c);
void orc_cache_destroy(orc_cache* c);
/* Copy cached keys/values of (layer, head) for positions [0, len) into out [len*head_dim]. */
int orc_cache_read(const orc_cache* c, size_t layer, size_t head, int values, float* out);

int orc_forward(const orc_model* m, const uint32_t* ids, size_t n, float* logits, char* err);
int orc_forward_cached(const orc_model* m, orc_cache* c, const uint32_t* ids, size_t n, float* logits, char* err);
/* Greedy loops (temperature <= 0). out receives n + max_new ids. */
int orc_generate_cached(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out,
                        char* err);
int orc_generate(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out, char* err);
/* generate_cached that also writes, for each greedy step s, the top-1 minus
 * top-2 logit of the row it chose from into gaps[s] (max(1, max_new) floats). */
int orc_generate_cached_gaps(const orc_model* m, const uint32_t* prompt, size_t n, size_t max_new, uint32_t* out,
                             float* gaps, char* err);
float orc_top2_gap(const float* data, size_t n);

#ifdef __cplusplus
}
#endif
#endif
