// Persistent decode kernel instances for width 768, vocabulary 50257.
#include "decode_persistent_kernel.h"

namespace rtg {
namespace pk {
const void* kernel_768_50257_f32() { return (const void*)decode_step_kernel<768, 50257, W_F32>; }
const void* kernel_768_50257_bf16() { return (const void*)decode_step_kernel<768, 50257, W_BF16>; }
}  // namespace pk
}  // namespace rtg
