// Elementwise device functions shared by the stream kernels and the fused GEMM
// epilogues, so a fused and an unfused evaluation run the same instructions
// and give the same bits.
#pragma once

#include <hip/hip_runtime.h>

namespace jade {
namespace hipk {

// SwiGLU with the reference's stable sigmoid (src/runtime/ir.rs:487):
// e = exp(-|g|), sigmoid = g >= 0 ? 1/(1+e) : e/(1+e), out = (g * sigmoid) * u.
__device__ inline float swiglu(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-fabsf(g) * 1.44269504088896340736f);
    const float sigmoid = g >= 0.f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return (g * sigmoid) * u;
}

}  // namespace hipk
}  // namespace jade
