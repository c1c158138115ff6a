// Tiled persistent decode step (decode_tile_kernel.h): plan and launch.
// Included by the .hip host files only (it carries the kernel's parameter
// types).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "decode_persistent.h"
#include "decode_tile_kernel.h"

namespace rtg {

struct TilePlan {
  void* arena = nullptr;  // weight tiles, folded constants, LM-head constants
  tk::TLayer* layers_dev = nullptr;
  tk::TParams base{};     // model-wide fields; per-cache fields are filled by the state
  size_t tag_words = 0;   // tagged exchange words of one cache
  const void* kernel = nullptr;
};

// Shapes the tiled step is built for: f32 weights, d = 768 (GPT-2 small's
// width), the GPT-2 vocabulary, 256 CUs.
bool tile_supported(int d, int H, int V, int wtype, int cus);
TilePlan* tile_plan_create(const PersistentWeights& w);
void tile_plan_destroy(TilePlan* tp);
// Longest context (positions including the new token) the tiled step takes.
int tile_max_len();
hipError_t tile_decode_step(const TilePlan* tp, const tk::TParams& p, hipStream_t stream, bool cooperative);

}  // namespace rtg
