/* rtgpu: MI355X (gfx950) GPT-2 token loop behind a C ABI.
 *
 * Each entry point mirrors one item of rusttorch's public GPT-2 API
 * (rusttorch-core/src/nn/gpt2.rs, re-exported at nn/mod.rs:50,94) and follows
 * the conventions of rusttorch's own C ABI (rusttorch-core/src/ffi/):
 * fallible calls return rtg_result {success, error_msg} like CResult
 * (ffi/tensor.rs:37-64); the message is owned by the library and released
 * with rtg_free_error_message (ffi/tensor.rs:66-72); host buffers are
 * caller-allocated and results are written into them (ffi/ops.rs:26-39).
 * Error strings are the reference's own (gpt2.rs:224-228, 269-279, 364-374,
 * 616-618).
 *
 * Threading: a model is immutable after construction and may be shared by
 * threads (gpt2.rs:358 takes &self); a cache binds one HIP stream and must not
 * be used from two threads at once (gpt2.rs:361 takes &mut KVCache). All calls
 * are synchronous from the host's point of view, as in the reference.
 *
 * There is no CPU fallback: creating a model without a usable gfx950 device
 * fails with an error. */
#ifndef RTGPU_H
#define RTGPU_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CResult, ffi/tensor.rs:37-64. */
typedef struct {
  bool success;
  char* error_msg; /* NULL on success; free with rtg_free_error_message */
} rtg_result;

/* Gpt2Config, gpt2.rs:82-104. The fields are public in the reference, which
 * takes head_dim = n_embd / n_head (gpt2.rs:349-352). This build accepts the
 * configurations its kernels are written for and refuses the others when the
 * model is created, before anything is uploaded, with these errors:
 *   "n_embd <d> is not divisible by n_head <h>"   (the reference would
 *       truncate head_dim and read past its rows)
 *   "head_dim <hd> > 64 is not supported"         (head_dim <= 64 only)
 *   "n_embd <d> must be a multiple of 8"          (16-byte row vectors)
 * Every GPT-2 checkpoint (head_dim 64, n_embd 768 / 1024 / 1280 / 1600) and
 * the reference's own test configuration (n_embd 8, 2 heads) are accepted.
 * The fastest batch-1 decode step (one persistent kernel per token) is built
 * for n_embd 128 with vocab_size <= 512, and for vocab_size <= 50257 at
 * n_embd 768 and 1024 (f32 and bf16 storage), 1280 (f32) and 1600 (bf16);
 * other accepted shapes decode through the batched step's kernel graph at
 * batch 1 (same results within the logits tolerance, about 4.5 us per kernel
 * launch, 5 launches per layer: GPT-2 XL in f32 takes 2.19 ms per token that
 * way, against 1.67 ms for XL bf16 on the persistent step). */
typedef struct {
  size_t vocab_size;
  size_t n_positions;
  size_t n_embd;
  size_t n_layer;
  size_t n_head;
  float layer_norm_epsilon;
} rtg_config;

/* GenerationConfig, gpt2.rs:31-79, plus the seed of the sampler (the
 * reference draws from rand::thread_rng, gpt2.rs:978,1005, so its sampled ids
 * are not reproducible; greedy decoding ignores the seed). */
typedef struct {
  size_t max_new_tokens;
  float temperature;
  size_t top_k;
  float top_p;
  float repetition_penalty;
  uint64_t seed;
} rtg_gen_config;

/* Element type of a host tensor handed to rtg_model_from_host; decoded to
 * f32 as safetensors.rs:232-348 does (BF16 = bits << 16, :389-391). */
typedef enum { RTG_F32 = 0, RTG_BF16 = 1, RTG_F16 = 2, RTG_F64 = 3 } rtg_dtype;

/* How the weights are held in HBM. RTG_STORE_BF16 keeps GEMM/GEMV weights as
 * bfloat16 (round-to-nearest-even) and upcasts them in-kernel; the oracle is
 * fed the same rounded values. */
typedef enum { RTG_STORE_F32 = 0, RTG_STORE_BF16 = 1 } rtg_storage;

/* One StateDict entry (nn/state_dict.rs:35-56): name, dtype, shape, data. */
typedef struct {
  const char* name;
  const void* data;
  rtg_dtype dtype;
  size_t ndim;
  const size_t* shape;
} rtg_named_tensor;

typedef struct rtg_model rtg_model;
typedef struct rtg_cache rtg_cache;

/* Device-event timings of a generate call (HIP events on the cache's stream).
 * profile_kernels is an input: when nonzero and the decode step is the single
 * persistent kernel, the decode steps are replayed once more launch by launch
 * (identical inputs and results) with events around that kernel, filling
 * decode_kernel_ms / decode_kernel_launches. */
typedef struct {
  int profile_kernels;
  double prefill_ms;     /* forward_cached over the prompt + first argmax */
  double decode_ms;      /* the (max_new - 1) single-token steps */
  size_t decode_steps;
  double decode_kernel_ms;       /* summed duration of the decode-step kernel */
  size_t decode_kernel_launches;
} rtg_timing;

/* rusttorch_init / rusttorch_cleanup / rusttorch_version, ffi/mod.rs:24-48. */
void rtg_init(void);
void rtg_cleanup(void);
const char* rtg_version(void);
/* rusttorch_free_error_message, ffi/tensor.rs:66-72. */
void rtg_free_error_message(char* msg);

/* Gpt2Model::from_safetensors, gpt2.rs:214-220 (F32/F64/F16/BF16 tensors).
 * Error: "Failed to load safetensors: ..." or "Missing weight: <name>". */
rtg_result rtg_model_from_safetensors(const char* path, const rtg_config* cfg, rtg_storage storage,
                                      rtg_model** out);
/* Gpt2Model::from_state_dict, gpt2.rs:223-263. Tensors use the reference's
 * Conv1D layout [in, out]; the data is copied (uploaded) before returning. */
rtg_result rtg_model_from_host(const rtg_config* cfg, const rtg_named_tensor* tensors, size_t n,
                               rtg_storage storage, rtg_model** out);
void rtg_model_destroy(rtg_model* model);
/* Gpt2Model::num_parameters, gpt2.rs:541-563. */
size_t rtg_num_parameters(const rtg_model* model);

/* Gpt2Model::new_cache / KVCache::new, gpt2.rs:349-352, 125-134. The cache
 * holds `batch` sequences and preallocates n_layer*batch*2*n_head*n_positions*
 * head_dim f32 in HBM. batch = 1 is the reference's cache. */
rtg_result rtg_cache_new(const rtg_model* model, size_t batch, rtg_cache** out);
/* KVCache::len / is_empty / clear, gpt2.rs:137-161. */
size_t rtg_cache_len(const rtg_cache* cache);
bool rtg_cache_is_empty(const rtg_cache* cache);
void rtg_cache_clear(rtg_cache* cache);
void rtg_cache_destroy(rtg_cache* cache);
/* Copies cached keys (values != 0: values) of one layer/head/sequence for
 * positions [0, len) to out[len * head_dim]; a test hook with no reference
 * counterpart (the reference's LayerKVCache fields are private). */
rtg_result rtg_cache_read(const rtg_cache* cache, size_t layer, size_t head, size_t seq, int values, float* out);

/* Gpt2Model::forward, gpt2.rs:269-304: logits_out[n * vocab_size]. */
rtg_result rtg_forward(const rtg_model* model, const uint32_t* ids, size_t n, float* logits_out);
/* Gpt2Model::forward_cached, gpt2.rs:358-399: logits_out[n * vocab_size]
 * (may be NULL to skip the device-to-host copy). The cache must have batch 1
 * and belong to model. One new token (n == 1) runs the persistent decode
 * step that generate_cached runs per token, where the model's shape has one;
 * 2..32 tokens run the multi-row forward in one launch (f32 weights, n_embd
 * 128, 768 or 1024); more tokens run the prefill kernels. */
rtg_result rtg_forward_cached(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                              float* logits_out);
/* forward_cached without device allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments as rtg_forward_cached and the kernels of its path for n >= 2
 * (the same results bit for bit; for n == 1 rtg_forward_cached runs the
 * persistent decode step instead, and the two agree within the logits
 * tolerance), but the pass's work rows and logits live in a fixed scratch
 * array of 16 MiB + 64 KiB per device inside the library instead of the
 * cache's buffers, and nothing is allocated. Up to 32 tokens run the
 * multi-row forward (its flags and epoch in the 64 KiB, kept between calls);
 * more run the prefill kernels, with the limit: n * (10 * n_embd +
 * vocab_size) floats (each of the six parts rounded up to 64) must fit in
 * 16 MiB, e.g. n <= 72 for GPT-2 small, n <= 63 for XL; a larger n returns
 * an error. The prefill GEMMs' split-k partials take what is left of the
 * array; where they do not fit the GEMMs run unsplit. All calls on one
 * device share the array and take turns on it (a per-device lock held until
 * the call's stream has drained). The cache must belong to model. */
rtg_result rtg_forward_cached_noalloc(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                                      float* logits_out);
/* Gpt2Model::generate (uncached, sliding window), gpt2.rs:311-346.
 * out receives n + max_new ids. */
rtg_result rtg_generate(const rtg_model* model, const uint32_t* prompt, size_t n, size_t max_new,
                        float temperature, uint64_t seed, uint32_t* out);
/* Gpt2Model::generate_cached, gpt2.rs:405-441. out receives n + max(1, max_new)
 * ids: like the reference, the prefill token is appended even if max_new == 0. */
rtg_result rtg_generate_cached(const rtg_model* model, const uint32_t* prompt, size_t n, size_t max_new,
                               float temperature, uint64_t seed, uint32_t* out);
/* Gpt2Model::generate_with_config, gpt2.rs:447-474 (+ sample_logits :871-906).
 * out receives n + max(1, cfg->max_new_tokens) ids. Non-greedy token choice
 * runs on the device for vocab_size <= 65536 (every GPT-2 vocabulary);
 * beyond it the call returns "vocabulary too large for the device sampler". */
rtg_result rtg_generate_with_config(const rtg_model* model, const uint32_t* prompt, size_t n,
                                    const rtg_gen_config* cfg, uint32_t* out);

/* Batched extension (new API: the reference is batch-1 only; its oracle for
 * batch B is B independent calls). ids/prompts are [batch][n] row-major. */
rtg_result rtg_forward_cached_batched(const rtg_model* model, rtg_cache* cache, const uint32_t* ids, size_t n,
                                      float* logits_out /* [batch][n][V] or NULL */);
/* Greedy generate_cached over `batch` equal-length prompts; out is
 * [batch][n + max(1, max_new)]. timing may be NULL. */
rtg_result rtg_generate_cached_batched(const rtg_model* model, const uint32_t* prompts, size_t batch, size_t n,
                                       size_t max_new, uint32_t* out, rtg_timing* timing);

/* ---- BpeTokenizer, rusttorch-core/src/data/tokenizer.rs (host-side text in
 * and out; used by the reference's example at examples/gpt2.rs:77-95).
 * Text is UTF-8 with an explicit length (a Rust &str). Buffers that a call
 * returns (ids, text, spans) are owned by the caller and released with
 * rtg_free_buffer. Errors carry the reference's messages. ---- */
typedef struct rtg_tokenizer rtg_tokenizer;
/* BpeTokenizer::from_files, tokenizer.rs:45-53. Errors: "Failed to read
 * vocab.json: <io error>", "Failed to read merges.txt: <io error>", then those
 * of from_strings. */
rtg_result rtg_tokenizer_from_files(const char* vocab_json_path, const char* merges_txt_path, rtg_tokenizer** out);
/* BpeTokenizer::from_strings, tokenizer.rs:55-82 (parse_vocab_json :356-401,
 * parse_merges :486-514). */
rtg_result rtg_tokenizer_from_strings(const char* vocab_json, size_t vocab_len, const char* merges_txt,
                                      size_t merges_len, rtg_tokenizer** out);
/* BpeTokenizer::from_vocab_and_merges, tokenizer.rs:186-219: token i gets id
 * i, merge rule r gets rank r. Strings are NUL-terminated UTF-8. */
rtg_result rtg_tokenizer_from_vocab_and_merges(const char* const* vocab, size_t n_vocab, const char* const* merge_a,
                                               const char* const* merge_b, size_t n_merges, rtg_tokenizer** out);
void rtg_tokenizer_destroy(rtg_tokenizer* t);
/* BpeTokenizer::encode, tokenizer.rs:85-112: *ids receives *n token ids. */
rtg_result rtg_tokenizer_encode(const rtg_tokenizer* t, const char* text, size_t len, uint32_t** ids, size_t* n);
/* BpeTokenizer::decode, tokenizer.rs:115-130: *text receives *len bytes of
 * UTF-8 (from_utf8_lossy), NUL-terminated. */
rtg_result rtg_tokenizer_decode(const rtg_tokenizer* t, const uint32_t* ids, size_t n, char** text, size_t* len);
/* BpeTokenizer::vocab_size / token_to_id / id_to_token, tokenizer.rs:133-145.
 * id_to_token points *token at the tokenizer's own copy (valid while it
 * lives); false is Rust's None. */
size_t rtg_tokenizer_vocab_size(const rtg_tokenizer* t);
bool rtg_tokenizer_token_to_id(const rtg_tokenizer* t, const char* token, size_t len, uint32_t* id);
bool rtg_tokenizer_id_to_token(const rtg_tokenizer* t, uint32_t id, const char** token, size_t* len);
/* pre_tokenize, tokenizer.rs:260-331 (private in the reference; exported for
 * the parity tests): byte ranges of the words, (*spans)[2k] .. (*spans)[2k+1]. */
rtg_result rtg_tokenizer_pre_tokenize(const char* text, size_t len, size_t** spans, size_t* n_words);
/* build_byte_encoder, tokenizer.rs:223-241 (private in the reference;
 * exported for the parity tests): the code point of every byte. */
void rtg_tokenizer_byte_encoder(uint32_t out[256]);
/* Releases a buffer returned by rtg_tokenizer_encode / _decode / _pre_tokenize. */
void rtg_free_buffer(void* p);

#ifdef __cplusplus
}
#endif
#endif /* RTGPU_H */
