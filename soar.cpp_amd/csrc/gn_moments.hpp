// gn_moments.hpp - the block-level combine of shifted sums into (mean, M2),
// shared by the GroupNorm statistics pass (k_stats) and the convolution
// epilogues that produce the same chunk partials, so both combine their
// threads' sums with the same float64 operations in the same order; and
// the backward finish's per-plane and per-unit sums, shared by its own
// finish blocks and the fused CBA backward kernels that fold it.
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

// ---- the GroupNorm backward finish's sums ----------------------------
// Each plane's (sum dz, sum dz xhat) comes from its cpp chunk partials of
// the reduction pass, added by a group of gs lanes (gs the power of two at
// or above cpp, at most 64): lane r adds partials r, r + gs, ... in order,
// then an xor butterfly over the group.  The result depends on cpp alone,
// not on which group or block adds the plane, so a consumer that folds the
// finish gets the finish's own bits.
constexpr int kBwdFinishThreads = 256;  // threads of a finish block

__device__ __forceinline__ int bwd_plane_lanes(int cpp) {
    int gs = 1;
    while (gs < 64 && gs < cpp) gs <<= 1;
    return gs;
}

// The plane's sums in every lane of the group (lane r of gs); `live`
// false: zeros (the group still takes part in the butterfly).
__device__ __forceinline__ double2 bwd_plane_sum(const double2* __restrict__ pp, int cpp,
                                                 int gs, int r, bool live) {
    double A = 0.0, B = 0.0;
    if (live) {
        int q = r;
        for (; q + 3 * gs < cpp; q += 4 * gs) {
            const double2 v0 = pp[q], v1 = pp[q + gs], v2 = pp[q + 2 * gs], v3 = pp[q + 3 * gs];
            A += v0.x;
            B += v0.y;
            A += v1.x;
            B += v1.y;
            A += v2.x;
            B += v2.y;
            A += v3.x;
            B += v3.y;
        }
        for (; q < cpp; q += gs) {
            const double2 v = pp[q];
            A += v.x;
            B += v.y;
        }
    }
    for (int off = gs >> 1; off > 0; off >>= 1) {
        A += __shfl_xor(A, off);
        B += __shfl_xor(B, off);
    }
    return make_double2(A, B);
}

// Sums of planes plane0 + j, j < J, into ps[j] (shared memory), by the
// block's NT threads in groups of gs lanes; with pgam, also gamma of each
// plane's channel (1 without gamma) into pgam[j], loaded with the partials
// so bwd_unit_sums waits for no further load.  The reduction's partials
// number below 2^31 (its grid), so 32-bit indices.  No synchronisation.
template <int NT>
__device__ __forceinline__ void bwd_plane_sums(const double2* __restrict__ part, int plane0,
                                               int J, int cpp, double2* ps,
                                               const float* __restrict__ gamma = nullptr,
                                               int C = 1, float* pgam = nullptr) {
    const int gs = bwd_plane_lanes(cpp);
    const int ngroups = NT / gs;
    const int grp = (int)threadIdx.x / gs, r = (int)threadIdx.x & (gs - 1);
    for (int j = grp; j - grp < J; j += ngroups) {
        const bool live = j < J;
        const int plane = plane0 + (live ? j : 0);
        float gj = 1.0f;
        if (pgam && live && r == 0 && gamma) gj = gamma[(unsigned)plane % (unsigned)C];
        const double2 ab = bwd_plane_sum(part + (unsigned)plane * (unsigned)cpp, cpp, gs, r, live);
        if (live && r == 0) {
            ps[j] = ab;
            if (pgam) pgam[j] = gj;
        }
    }
}

// (S1, S2) = sum_j gamma_j (A_j, B_j) of a unit from its planes' sums
// ps[0..cpg) and their channels' gamma pgam[0..cpg), in the finish block's
// order: each of its kBwdFinishThreads / gs groups adds its planes j,
// j + ngroups, ... from zero, then the groups are added in order.  One
// thread.
__device__ __forceinline__ double2 bwd_unit_sums(const double2* ps, const float* pgam, int cpg,
                                                 int cpp) {
    const int ngroups = kBwdFinishThreads / bwd_plane_lanes(cpp);
    double s1 = 0.0, s2 = 0.0;
    for (int g = 0; g < ngroups && g < cpg; ++g) {
        double S1 = 0.0, S2 = 0.0;
        for (int j = g; j < cpg; j += ngroups) {
            const double gj = (double)pgam[j];
            S1 += gj * ps[j].x;
            S2 += gj * ps[j].y;
        }
        s1 += S1;
        s2 += S2;
    }
    return make_double2(s1, s2);
}

}  // namespace gn
}  // namespace soar
