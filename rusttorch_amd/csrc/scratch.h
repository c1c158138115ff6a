// Device scratch for the entry point that allocates nothing
// (rtg_forward_cached_noalloc): one fixed array per device, in the library's
// code object, holding the activations and logits of one forward pass.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include <mutex>

namespace rtg {

// 16 MiB: GPT-2 small takes (10 d + V) floats per new token (x, ln, att:
// d each; qkv 3d; h 4d; one logits row), so 72 tokens fit; XL 63. The
// prefill GEMMs' split-k partials use what is left, else the GEMMs run
// unsplit.
constexpr size_t kScratchFloats = (size_t)4 << 20;
// The array also holds, ahead of those 16 MiB, 64 KiB that only the multi-row
// forward (short prompts, rows.h) uses: its flag words, epoch and counters,
// which must keep what its previous launch on this device left (zeros before
// the first). Its work rows and logits then take the 16 MiB that follow.
constexpr size_t kScratchHeadFloats = (size_t)16 << 10;

// Device address of `device`'s copy of the array (looked up once per device
// with hipGetSymbolAddress, with that device current, which also clears the
// 64 KiB head; the current device is restored afterwards). Null with *err set
// on failure. The 16 MiB of activations start kScratchHeadFloats after it.
float* scratch_device_ptr(int device, hipError_t* err);

// Held by a call from its first use of `device`'s array until its stream has
// drained, so that calls from several threads take turns on the array.
std::mutex& scratch_lock(int device);

}  // namespace rtg
