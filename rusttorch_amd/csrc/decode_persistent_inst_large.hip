// Persistent decode kernel instances for GPT-2 large (f32) and XL (bf16 weights).
#include "decode_persistent_kernel.h"

namespace rtg {
namespace pk {
const void* kernel_1280_50257_f32() { return (const void*)decode_step_kernel<1280, 50257, W_F32>; }
const void* kernel_1600_50257_bf16() { return (const void*)decode_step_kernel<1600, 50257, W_BF16>; }
}  // namespace pk
}  // namespace rtg
