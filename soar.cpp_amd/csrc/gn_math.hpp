// gn_math.hpp - the SiLU arithmetic shared by every kernel that applies or
// differentiates it, so that a fused kernel recomputes bit for bit what the
// stand-alone GroupNorm passes compute; and the block barrier of kernels
// whose waves hand data to each other through LDS only.
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

// Block barrier that orders LDS accesses only.  __syncthreads() is a
// workgroup-scope release/acquire, which also waits for the wave's global
// stores to complete (s_waitcnt vmcnt(0)) before the barrier: in a loop
// that stores results every step that wait puts a store round trip on each
// step.  Here the fences are limited to the local (LDS) address space, so
// the wait is for LDS accesses alone; global memory written before the
// barrier is not made visible to the block by it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace gn
}  // namespace soar
