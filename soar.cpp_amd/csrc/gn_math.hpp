// gn_math.hpp - the SiLU arithmetic shared by every kernel that applies or
// differentiates it, so that a fused kernel recomputes bit for bit what the
// stand-alone GroupNorm passes compute.
#pragma once

#include <hip/hip_runtime.h>

namespace soar {
namespace gn {

constexpr float kLog2e = 1.4426950408889634f;

// sigmoid(z) = 1/(1+exp(-z)) with the hardware 2^x (v_exp_f32) and
// reciprocal (v_rcp_f32).  exp overflow to +inf gives 0, underflow gives 1.
__device__ __forceinline__ float sigmoid_fast(float z) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * kLog2e));
}

__device__ __forceinline__ float silu_fast(float z) { return z * sigmoid_fast(z); }

// Gradient at the SiLU input: g * s * (1 + z*(1-s)), s = sigmoid(z).
__device__ __forceinline__ float dsilu_fast(float g, float z) {
    float s = sigmoid_fast(z);
    return g * s * fmaf(z, 1.0f - s, 1.0f);
}

}  // namespace gn
}  // namespace soar
