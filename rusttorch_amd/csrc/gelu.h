// gelu_new (rusttorch-core/src/nn/gpt2.rs:837-847) of the prefill GEMM
// epilogues and the multi-row forward.
#pragma once
#include <hip/hip_runtime.h>

namespace rtg {

// The reference's association for the inner term. Since tanh(y) = 1 - 2 /
// (e^(2y) + 1), 0.5 x (1 + tanh(y)) equals x / (1 + e^(-2y)): one hardware
// exp2 (v_exp_f32) and one reciprocal instead of the libm tanh sequence,
// within a few ulp of it; the limits are exact (e^(-2y) -> inf gives -0 / 0
// for x < 0 as the tanh form does, -> 0 gives x).
__device__ __forceinline__ float gelu_new(float x) {
  const float sqrt_2_pi = 0.7978845608028654f;  // (2.0f32 / PI).sqrt() rounded to f32
  const float inner = sqrt_2_pi * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(inner * -2.8853900817779268f);  // e^(-2 inner) = 2^(-2 log2(e) inner)
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace rtg
