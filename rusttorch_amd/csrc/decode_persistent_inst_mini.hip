// Persistent decode kernel instances for width 128, vocabulary 512.
#include "decode_persistent_kernel.h"

namespace rtg {
namespace pk {
const void* kernel_128_512_f32() { return (const void*)decode_step_kernel<128, 512, W_F32>; }
const void* kernel_128_512_bf16() { return (const void*)decode_step_kernel<128, 512, W_BF16>; }
}  // namespace pk
}  // namespace rtg
