// Packed 64-bit argmax key for argmax_f32 (rusttorch-core/src/nn/gpt2.rs:858-868),
// shared by every kernel that picks a greedy token (the argmax kernel, the
// batched LM-head epilogue, the persistent decode step and the sampler's
// greedy branch).
//
// The reference scans from best = -inf with a strict '>', so:
//   * the first index of the maximum wins (ties keep the earlier index);
//   * NaN and -inf never win; a row with nothing above -inf returns index 0;
//   * -0.0 and +0.0 compare equal, so between them the earlier index wins.
// Key = (orderable bits of v) << 32 | ~idx: a plain unsigned max over keys is
// the reference's scan in any reduction order. -0.0 is given +0.0's bits
// before packing (otherwise -0.0 would order below +0.0), and key 0 stands
// for "nothing above -inf" (every real key is > 0: the orderable bits of
// -FLT_MAX are 0x00800000).
//
// RTG_HD may be predefined (e.g. as `inline`) to compile this header in a
// host-only unit test.
#pragma once
#include <stdint.h>

#ifndef RTG_HD
#define RTG_HD __host__ __device__ __forceinline__
#endif

namespace rtg {

RTG_HD uint64_t argmax_key(float v, uint32_t idx) {
  if (!(v > -__builtin_inff())) return 0ull;  // -inf and NaN never win
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (b == 0x80000000u) b = 0u;  // -0.0 ties with +0.0
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint64_t)(~idx);
}

// Index of the winning key; key 0 (no value above -inf) gives index 0, the
// reference's initial best_idx.
RTG_HD uint32_t argmax_key_index(uint64_t key) { return key == 0ull ? 0u : ~(uint32_t)(key & 0xffffffffull); }

}  // namespace rtg
