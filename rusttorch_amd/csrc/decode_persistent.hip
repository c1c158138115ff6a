// Persistent decode step: not enabled yet (the multi-kernel decode graph runs).
#include "decode_persistent.h"

namespace rtg {

struct PersistentPlan {
  PersistentWeights w;
};
struct PersistentState {
  int unused;
};

PersistentPlan* persistent_plan_create(const PersistentWeights& w) { return new PersistentPlan{w}; }
void persistent_plan_destroy(PersistentPlan* p) { delete p; }
bool persistent_supported(const PersistentPlan*, int) { return false; }
PersistentState* persistent_state_create(PersistentPlan*, float*, float*, int, uint32_t*, int*, float*,
                                         unsigned long long*) {
  return nullptr;
}
void persistent_state_destroy(PersistentState* s) { delete s; }
void persistent_decode_step(PersistentState*, hipStream_t) {}

}  // namespace rtg
