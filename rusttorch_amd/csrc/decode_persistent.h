// Persistent single-launch decode step (one kernel per generated token) for
// batch 1; see decode_persistent.hip for the design.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
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
                                         unsigned long long* keys, uint32_t* ids_dev, int* step_dev);
void persistent_state_destroy(PersistentState* s);
// Enqueue one decode step: reads *token_dev / *pos_dev, writes the logits,
// and finishes the step itself (the finalize kernel's work): the argmax token
// goes to *token_dev and ids_dev[*step_dev], *pos_dev and *step_dev advance
// by one, the packed argmax key is cleared.
// pos is the position of the token the step consumes (the value *pos_dev
// holds when the step runs), or -1 if unknown: it selects between the
// tiled step (short contexts, where built) and the row-split step.
// The caller must hold persistent_launch_lock(device) from the first step it
// enqueues until its stream has drained.
hipError_t persistent_decode_step(PersistentState* s, hipStream_t stream, bool cooperative, int pos);
// One lock per device: persistent steps of two streams in flight at once could
// each hold part of the CUs and wait on workgroups that cannot start.
std::mutex& persistent_launch_lock(int device);
unsigned* persistent_epoch(PersistentState* s);
unsigned* persistent_err(PersistentState* s);
// Writes the latest step's per-workgroup timestamps to $RTG_TRACE_FILE (if set).
void persistent_dump_trace(PersistentState* s);

}  // namespace rtg
