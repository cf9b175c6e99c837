// gn_moments.hpp - the block-level combine of shifted sums into (mean, M2),
// shared by the GroupNorm statistics pass (k_stats) and the convolution
// epilogues that produce the same chunk partials, so both combine their
// threads' sums with the same float64 operations in the same order.
#pragma once

#include <hip/hip_runtime.h>

namespace soar {
namespace gn {

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off);
    return v;
}

// (mean, M2) from the sums about R over N elements: S = sum (x - R),
// Q = sum (x - R)^2.
__device__ __forceinline__ double2 centred_moments(double S, double Q, double N, double R) {
    const double m = S / N;
    return make_double2(R + m, fmax(Q - S * m, 0.0));
}

// The block's (mean, M2), valid in thread 0, from each thread's fp32 sums
// s = sum (x - K), q = sum (x - K)^2 over its cnt elements about its own
// shift K, without a division per thread or per step of the tree: each
// thread's sums are re-centred on its wave's reference Rw (lane 0's K; when
// lane 0 has no elements, no lane of the wave has) as S = n d + s,
// Q = q + d (2 s + n d) with d = K - Rw (the sums of x - Rw and of its
// square), the wave adds them, and thread 0 re-centres the waves' sums on
// wave 0's reference in wave order.  lds: 4 * NT / 64 doubles.  Ends with
// the block synchronised once (the caller synchronises before reusing lds).
template <int NT>
__device__ __forceinline__ double2 block_moments(float K, float s_f, float q_f, int cnt,
                                                 double* lds) {
    constexpr int W = NT / 64;
    const float Rw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(K)));
    double S = 0.0, Q = 0.0;
    if (cnt > 0) {
        const double s = (double)s_f;
        const double q = (double)q_f;
        const double d = (double)K - (double)Rw;
        const double nd = (double)cnt * d;
        S = nd + s;
        Q = fma(d, 2.0 * s + nd, q);
    }
    int n = cnt;
    n = wave_sum(n);
    S = wave_sum(S);
    Q = wave_sum(Q);
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    if (lane == 0) {
        lds[w] = (double)n;
        lds[W + w] = S;
        lds[2 * W + w] = Q;
        lds[3 * W + w] = (double)Rw;
    }
    __syncthreads();
    double2 r = make_double2(0.0, 0.0);
    if (t == 0) {
        const double R0 = lds[3 * W];
        double N = lds[0], S0 = lds[W], Q0 = lds[2 * W];
#pragma unroll
        for (int i = 1; i < W; ++i) {
            const double ni = lds[i], Si = lds[W + i];
            if (ni == 0.0) continue;
            const double d = lds[3 * W + i] - R0;
            const double nd = ni * d;
            Q0 += fma(d, 2.0 * Si + nd, lds[2 * W + i]);
            S0 += Si + nd;
            N += ni;
        }
        r = centred_moments(S0, Q0, N, R0);
    }
    return r;
}

}  // namespace gn
}  // namespace soar
