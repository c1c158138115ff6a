// Persistent batched decode step: one cooperative launch per generated token
// for 2..16 sequences (forward_cached with one new token per sequence plus
// the greedy choice, gpt2.rs:358-399, 431-437, 858-868); see bdecode.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bgemv.h"

namespace rtg {

constexpr int BD_G = 256;  // workgroups: one per CU of an MI355X

struct BdLayer {
  const void *qkv, *proj, *fc, *mproj;  // tile-ordered weights
  const float *cq, *sq, *cf, *sf;       // LN1 / LN2 folded into c_attn / c_fc
  const float *ln1w, *ln2w, *baproj, *bmproj;
};

struct BdPlans {
  BgemvPlan pq, pp, pf, pm, pl;  // c_attn, attn c_proj, c_fc, mlp c_proj, LM head (8 waves per unit)
};

struct BdParams {
  const BdLayer* layers;  // device array [L]
  int L, B, d, V, H, P, wtype;
  float eps;
  const void* wte;
  const float* wpe;
  const void* lm;  // tile-ordered wte (the tied LM head)
  const float *sl, *cl, *lnfw;
  float *kc, *vc;  // [L][B][H][P][64]
  long kv_layer;   // floats per layer
  float *x, *qkv, *att, *h, *logits;
  float* spart;   // LayerNorm statistics partials [groups][16][2]
  float* part;    // split-k partials
  unsigned* cnt;  // split-k counters (zeroed, left zeroed)
  unsigned* bar;  // barrier flags, one per workgroup 128 bytes apart
  unsigned bar_base;  // flag value reached before this step's first barrier
  unsigned* err;      // nonzero after a barrier wait timed out
  uint32_t* token;    // [B] current tokens in, argmax tokens out
  int* pos;           // position of the current tokens; advanced by one
  uint32_t* ids;      // [B][ld_ids] generated ids
  int* step;          // ids[b][*step] = token; advanced by one
  int ld_ids;
  unsigned long long* keys;  // [B] argmax keys (zeroed, left zeroed)
  unsigned* done;            // arrivals after the LM head (zeroed, left zeroed)
  BdPlans plan;
  // optional: workgroup 0 writes the 100 MHz clock after each grid barrier
  // and at the end of its LM head work (bd_barriers(L) + 2 entries)
  unsigned long long* trace;
};

// The work split of the persistent step for one GEMV shape.
BgemvPlan bd_plan(int N, int K, int wtype);
// Grid barriers in one step (bar_base advances by this much per launch):
// after the embedding and after each of the 5 phases of every layer.
__host__ __device__ inline int bd_barriers(int L) { return 1 + 5 * L; }
// Workspace sizes for a set of plans.
size_t bd_part_floats(const BdPlans& p);
size_t bd_groups(const BdPlans& p);
hipError_t launch_bdecode(const BdParams& p, hipStream_t s);

}  // namespace rtg
