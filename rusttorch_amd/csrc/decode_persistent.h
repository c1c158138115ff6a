// Persistent single-launch decode step (one kernel per generated token).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "../../include/rtgpu.h"

namespace rtg {

struct PersistentLayer {
  const void *wqkv, *waproj, *wfc, *wmproj;
  const float *bqkv, *baproj, *bfc, *bmproj, *ln1w, *ln1b, *ln2w, *ln2b;
};

struct PersistentWeights {
  rtg_config cfg;
  int wtype;
  const void* wte;
  const float *wpe, *lnfw, *lnfb;
  std::vector<PersistentLayer> layers;
};

struct PersistentPlan;
struct PersistentState;

PersistentPlan* persistent_plan_create(const PersistentWeights& w);
void persistent_plan_destroy(PersistentPlan* p);
bool persistent_supported(const PersistentPlan* p, int batch);
PersistentState* persistent_state_create(PersistentPlan* p, float* kcache, float* vcache, int batch,
                                         uint32_t* token_dev, int* pos_dev, float* logits,
                                         unsigned long long* keys);
void persistent_state_destroy(PersistentState* s);
void persistent_decode_step(PersistentState* s, hipStream_t stream);

}  // namespace rtg
