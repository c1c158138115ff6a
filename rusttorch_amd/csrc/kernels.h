// Launchers for the gfx950 kernels of the GPT-2 token loop.
//
// Device layouts (all row-major, all in HBM):
//   weights W^T [N][K]  : every Conv1D weight of the reference ([in=K][out=N],
//                         gpt2.rs:15-17) is stored transposed, so each output
//                         is a dot product over a contiguous K row.
//   wte [V][d]          : token table; also the tied LM head's W^T.
//   KV cache            : [layer][seq][head][n_positions][64] f32.
//   activations         : [rows][cols] f32, rows = seq * T + t.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rtg {

enum WType { W_F32 = 0, W_BF16 = 1 };

// GEMV / GEMM epilogues.
enum Epi {
  EPI_BIAS = 0,       // y = acc + bias
  EPI_BIAS_GELU = 1,  // y = gelu_new(acc + bias)
  EPI_BIAS_RESID = 2, // y = y + (acc + bias)          (in-place residual)
  EPI_NONE = 3,       // y = acc                        (LM head)
};

struct KvDst {
  float* k;        // cache keys base for this layer: [seq][head][P][64]
  float* v;
  int n_head;
  int n_pos;       // P
  int d;           // n_embd
};

// Input layout of the batched decode GEMV (bgemv.hip): element (m, k) of an
// M-row input read in k-tiles of tk columns (16 for f32 weights, 32 for bf16)
// sits at [k / tk][chunk][m][k % 4], with the 4-column chunks c = (k % tk) / 4
// of a tile in the order the GEMV's lanes load them (for tk = 32, lane group
// g of 16 lanes holds columns 8g..8g+7 and loads them as two 16-byte halves,
// so the half-h chunks of all groups come first). One 16-byte load of a lane
// group then reads M rows of one chunk contiguously. M = 1 is row order.
__host__ __device__ inline size_t xt_index(int m, int k, int M, int tk) {
  const int c = (k % tk) >> 2;
  const int pos = tk == 32 ? ((c & 1) << 2) | (c >> 1) : c;
  return ((size_t)(k / tk) * (tk >> 2) + pos) * (size_t)M * 4 + (size_t)m * 4 + (k & 3);
}

// Token + position embedding. ids[rows]; position of row r = pos0 + (r % T),
// or, when pos_dev != nullptr, *pos_dev (decode: T == 1).
void launch_embed(hipStream_t s, const void* wte, int wtype, const float* wpe, const uint32_t* ids, int rows, int T,
                  int pos0, const int* pos_dev, int d, float* x);

// Row LayerNorm (gpt2.rs:636-666), rows x d.
void launch_layernorm(hipStream_t s, const float* x, const float* w, const float* b, float eps, int rows, int d,
                      float* out);

// Decode GEMV: y[b][n] = epi(sum_k x[b][k] * W[n][k]) for b < B (any B: more
// than 16 sequences run as slices of 16).
void launch_gemv(hipStream_t s, int B, const void* W, int wtype, const float* bias, const float* x, int ldx,
                 float* y, int ldy, int N, int K, int epi);
// Decode QKV GEMV: q part to q[b][d]; k/v parts into the cache at *pos_dev.
void launch_gemv_qkv(hipStream_t s, int B, const void* W, int wtype, const float* bias, const float* x, int ldx,
                     float* q, int ldq, int d, KvDst kv, const int* pos_dev);

// Decode attention over the cache for positions [0, *pos_dev] (gpt2.rs:772-834),
// one new token per sequence. out[b][ldo] rows, or with out_tk > 0 (head_dim
// 64 only) the GEMV input layout xt_index(b, col, B, out_tk).
void launch_attn_decode(hipStream_t s, int B, const float* q, int ldq, const float* kc, const float* vc,
                        int n_head, int n_pos, const int* pos_dev, float* out, int ldo, int out_tk = 0);

// Greedy argmax over rows of logits (gpt2.rs:858-868) into packed keys.
void launch_argmax(hipStream_t s, const float* logits, long ld, int rows, int V, unsigned long long* keys);
// Decode bookkeeping: token[b] = unpack(keys[b]); ids_out[b*ld + *step_dev] = token;
// keys reset; *pos_dev += 1; *step_dev += 1; *epoch += 1 when given.
void launch_finalize(hipStream_t s, int B, unsigned long long* keys, uint32_t* token, uint32_t* ids_out, int ld_ids,
                     int* pos_dev, int* step_dev, unsigned* epoch = nullptr);
// Extract tokens from keys without touching counters (prefill).
void launch_keys_to_tokens(hipStream_t s, int B, unsigned long long* keys, uint32_t* token);
void launch_reset_keys(hipStream_t s, int B, unsigned long long* keys);

// Prefill GEMM on MFMA: C[M][N] = epi(A[M][K] * W[N][K]^T); C row stride ldc.
// ws (ws_floats floats, may be null) holds split-k partial tiles: shapes with
// too few output tiles to fill the GPU split k when it is large enough
// (gemm_splitk_ws_floats), otherwise they run unsplit.
void launch_gemm(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias, float* C,
                 long ldc, int M, int N, int K, int epi, float* ws = nullptr, size_t ws_floats = 0);
// Workspace floats launch_gemm / launch_gemm_qkv use to split an M x N x K
// GEMM over k (0: it runs unsplit).
size_t gemm_splitk_ws_floats(int M, int N, int K);
// Prefill: append k/v columns of qkv [S*T][3d] into the cache at past.. past+T.
void launch_kv_append(hipStream_t s, const float* qkv, int S, int T, int past, KvDst kv);
// Prefill c_attn: C = A W^T + bias with the k/v columns ([d, 3d)) of row
// s*T + t written into the cache at position past + t instead of C (the
// append of LayerKVCache::append, gpt2.rs:500-514, in the GEMM's epilogue).
// Falls back to launch_gemm + launch_kv_append where the fused kernels do not
// apply (they need K % 64 == 0, 16-byte aligned operands and more than 64
// rows; f32 or bf16 weights).
void launch_gemm_qkv(hipStream_t s, const float* A, int lda, const void* W, int wtype, const float* bias, float* C,
                     long ldc, int M, int K, int S, int T, int past, KvDst kv, float* ws = nullptr,
                     size_t ws_floats = 0);
// Prefill causal attention for S sequences of T new tokens at offset past.
void launch_attn_prefill(hipStream_t s, const float* qkv, int S, int T, int past, const float* kc, const float* vc,
                         int n_head, int n_pos, int d, float* out);

// LayerNorm folded into the GEMV that follows it (computed once per model,
// accumulated in double): for output row r of W^T[N][K],
// s[r] = sum_k W[r][k] g[k] and c[r] = bias[r] + sum_k W[r][k] b[k]
// (bias may be null), so LN(x) W + bias = inv_std (W (x g) - mean s) + c.
bool ln_fold(const void* W, int wtype, int N, int K, const float* g, const float* b, const float* bias, float* s,
             float* c);

// bf16 conversion / transposition used once at model load.
// Token choice of one decode step on the device (sampling.hip).
struct SampleParams {
  float temperature;  // <= 0: greedy (argmax after the repetition penalty)
  int top_k;          // 0 or >= V: off
  float top_p;        // outside (0, 1): off
  float penalty;      // 1: off
  uint64_t seed;      // SplitMix64 seed; the draw of generation index g is number draw0 + g + 1
  uint32_t draw0;
};
// Picks the token of generation index g = *step_dev - 1 from logits[V] (the
// history is prompt[0, n_prompt) then ids[0, g)) and writes it to *token and
// ids[g]. One workgroup, no scratch memory. False when V is too large (> 65536).
bool launch_sample(hipStream_t s, const float* logits, int V, const uint32_t* prompt, int n_prompt, uint32_t* ids,
                   const int* step_dev, const SampleParams& sp, uint32_t* token);

// Element types of a source tensor as uploaded from the caller or the file.
enum { SRC_F32 = 0, SRC_BF16 = 1, SRC_F16 = 2 };
void launch_transpose_to(hipStream_t s, const void* src, int stype, int rows, int cols, void* dst, int wtype);
void launch_convert_to(hipStream_t s, const void* src, int stype, long n, void* dst, int wtype);

}  // namespace rtg
