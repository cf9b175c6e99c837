// gn_kernels.hip - fused GroupNorm(+SiLU) forward and backward for gfx950.
//
// The path is HBM-bound (about 1 flop per byte, no contraction), so every
// kernel is a streaming pass built for CDNA4's memory system:
//   * one 256-thread block (four wave64s) streams one contiguous chunk of
//     one (n, c) plane with 128-bit loads, four in flight per thread;
//   * per-block partial results go to a small workspace and are combined
//     in float64 in a fixed order by one "finish" block per unit, so results
//     are bitwise reproducible and no atomics or fences are used;
//   * the second pass (apply / dx) walks the chunks in reverse, so it
//     starts on what the first pass read last, still in the 256 MB MALL;
//   * units can be processed in batches (a tuning knob, off by default):
//     a batch's second pass then runs right after the first pass of the
//     next batch.  The finish blocks of batch b are the first blocks of the
//     first-pass kernel of batch b+1 (a kernel boundary makes batch b's
//     partials visible to them), so a batch costs two launches;
//   * per-block coefficients (mean, rstd, gamma, beta, S1, S2) are uniform
//     across the block and live in scalar registers;
//   * SiLU is recomputed in the backward from x and the saved statistics
//     instead of storing the pre-activation.
//
// Forward  (3 tensor passes): per batch k_stats (finish of the previous
//                             batch + partials), k_apply of the previous batch
// Backward (5 tensor passes): per batch k_bwd_reduce (finish of the previous
//                             batch + partials), k_bwd_dx of the previous
//                             batch; then k_param_finish for dgamma/dbeta
//
// Reference algorithms (pomagrenate/soar.cpp):
//   statistics  shaders/group_norm_stats.comp:25-73 (sum/sumsq, one
//               workgroup per group), src/cuda/ops/normalization_kernels.cu
//               :12-64 (Welford + Chan, one block per group),
//               src/nn/layers.cpp:690-710 (double sums).  Here: per-thread
//               shifted sums, combined across threads, blocks and chunks as
//               float64 sums re-centred on a data value (the Chan combine
//               unrolled); rstd = 1/sqrt(max(var,0)+eps), biased variance.
//   apply       shaders/group_norm_affine_silu.comp:33-65,
//               normalization_kernels.cu:70-91 + activation_kernels.cu:11-49,
//               layers.cpp:712-721,789-795.  Here (x-mean)*(gamma*rstd)+beta
//               (not the alpha*x+delta form, which loses digits when |mean|
//               is large), then z/(1+exp(-z)).
//   backward    layers.cpp:545-617 (GN) and :760-769 (SiLU),
//               normalization_kernels.cu:116-249.  Here one reduction pass
//               gives per-plane sum(dz) and sum(dz*xhat); dgamma/dbeta and
//               the per-group S1/S2 both derive from them.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "gn_internal.hpp"
#include "gn_math.hpp"
#include "gn_moments.hpp"
#include "soar_gn.h"
#include "xcd_order.hpp"

namespace soar {
namespace gn {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = kThreads / 64;

// Sum of (a, b) over a block of NT threads in a fixed order; valid in
// thread 0.  Ends with the block synchronised.
template <typename T, int NT = kThreads>
__device__ __forceinline__ void block_sum2(T& a, T& b, T* lds /*[2 * NT / 64]*/) {
    constexpr int W = NT / 64;
    a = wave_sum(a);
    b = wave_sum(b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) {
        lds[w] = a;
        lds[W + w] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        a = lds[0];
        b = lds[W];
#pragma unroll
        for (int i = 1; i < W; ++i) {
            a += lds[i];
            b += lds[W + i];
        }
    }
    __syncthreads();
}

// ---- re-centred moment sums (no division per term) -------------------
// Moments (n_k, mean_k, M2_k) about a common reference R: with
// d_k = mean_k - R,
//   S = sum n_k d_k,   Q = sum M2_k + n_k d_k^2,
// the combined mean is R + S/N and M2 = Q - S^2/N (N = sum n_k).  This is
// the Chan combine unrolled over all terms, as plain float64 sums in a
// fixed order; with R a value of the data (one partial's mean) every d_k is
// of the data's spread, so the final subtraction cancels nothing that
// matters.
__device__ __forceinline__ void centred_add(double& S, double& Q, double n, double mean,
                                            double m2, double R) {
    const double d = mean - R;
    const double nd = n * d;
    S += nd;
    Q += fma(nd, d, m2);
}


// Element count of chunk partial j of a unit (partials are plane-major,
// cpp per plane; only a plane's last chunk can be short).  j < 2^31: the
// plan keeps every grid below that.
__device__ __forceinline__ double partial_count(int64_t j, int64_t HW, int64_t chunk,
                                                int64_t cpp) {
    const int64_t k = (int64_t)((uint32_t)j % (uint32_t)cpp);
    return (double)min(chunk, HW - k * chunk);
}

// Chunk geometry of block `b`: plane index, element offset in the plane
// and length.
struct Chunk {
    int64_t plane, off, len;
};

__device__ __forceinline__ Chunk chunk_of(int64_t b, int64_t HW, int64_t chunk,
                                          int64_t cpp) {
    Chunk k;
    k.plane = b / cpp;
    k.off = (b - k.plane * cpp) * chunk;
    k.len = min(chunk, HW - k.off);
    return k;
}

// Block index of this block inside its batch [block0, block0 + nb): the
// XCD-aware order of xcd_block (each XCD runs 32 consecutive chunks), then
// reversed for the passes that walk back through the MALL.  Against the
// hardware order at config 3, statistics / apply / reduction / dx 163.7 /
// 336.8 / 319.1 / 508.3 -> 160.0 / 332.6 / 316.0 / 501.1 us, 1.326 ->
// 1.312 ms per step (three rounds, one box); with runs of 8 chunks per XCD
// the apply and the reduction had lost as much as the others gained.
__device__ __forceinline__ int64_t batch_block(int64_t block0, int64_t nb, int reverse) {
    const int64_t pb = xcd_block(blockIdx.x, nb);
    return block0 + (reverse ? nb - 1 - pb : pb);
}

// The same for the chunk blocks of a launch whose first fin_nu blocks
// finish the previous batch's units.
__device__ __forceinline__ int64_t chunk_block(int64_t block0, int64_t fin_nu) {
    return block0 + xcd_block((int64_t)blockIdx.x - fin_nu, (int64_t)gridDim.x - fin_nu);
}

template <bool NTL>
__device__ __forceinline__ f4 load4(const f4* p) {
    if (NTL) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ __forceinline__ void store4(f4* p, f4 v) {
    if (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

template <bool NT>
__device__ __forceinline__ void store1(float* p, float v) {
    if (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

// ======================================================================
// Forward pass 1: unit statistics of the previous batch, then per-chunk
// moments of this batch.
//
// Chunk blocks: each thread shifts its elements by its own first element K
// (so sums of d = x - K stay near the data's spread even when |mean| >>
// std), keeps fp32 sums of d and d*d in four independent lanes of
// accumulation, then the block combines them in float64 (re-centred sums,
// no division per thread).  part[b] = (mean, M2) of chunk b; its count is
// implied by the chunk geometry.
//
// Finish blocks (blockIdx.x < fin_nu): one per unit of the previous batch;
// combines the unit's cpg*cpp partials in a fixed order and writes mean and
// rstd.  The mean is also kept as hi + lo (hi = fp32 mean, lo = its fp32
// rounding residual): when std << |mean| the rounding of hi alone, times
// rstd, would shift xhat by up to ulp(mean)/2 * rstd, far above the 1e-4
// output tolerance.  lo goes to the caller's optional mean_lo (for the
// backward) and to the workspace (for the apply kernel of the same call).
// ======================================================================
// Element count of a unit's partial j: chunk partials (the statistics
// pass, the pointwise convolution's epilogue) ...
struct ChunkCount {
    int64_t HW, chunk, cpp;
    __device__ double operator()(int64_t j) const { return partial_count(j, HW, chunk, cpp); }
};

// ... or the depthwise forward's tile groups: partial j of a unit is group
// j % tpp of one of its planes, `rows` output rows (clipped at Ho) by 64
// columns (clipped at Wo); dw_stats_geometry's layout.
struct TileCount {
    int64_t tpp, tiles_x, rows, Ho, Wo;
    __device__ double operator()(int64_t j) const {
        const int64_t g = (int64_t)((uint32_t)j % (uint32_t)tpp);
        const int64_t ty = g / tiles_x, tx = g - ty * tiles_x;
        return (double)(min(rows, Ho - ty * rows) * min((int64_t)64, Wo - tx * 64));
    }
};

template <int NT = kThreads, typename Count>
__device__ void finish_unit(int64_t u, const double2* __restrict__ part, int64_t P,
                            const Count& count, double n_total, float* __restrict__ mean,
                            float* __restrict__ rstd, float* __restrict__ mean_lo,
                            float* __restrict__ lo_ws, float eps,
                            double* lds /*[2 * NT / 64]*/) {
    const int64_t first = u * P;
    // Sums about partial 0's mean (centred_add), each thread over partials
    // j, j + NT, ... in order, then the block in a fixed order.
    const double R = part[first].x;
    double S = 0.0, Q = 0.0;
    // Eight independent loads in flight per thread, then their sums in
    // index order (a load-add-load loop would wait a full memory latency
    // per partial).
    // (full batches carry no bounds test between the loads: a test per load
    // makes the compiler wait for each one)
    constexpr int kUnroll = 8;
    int64_t j0 = threadIdx.x;
    for (; j0 + (kUnroll - 1) * NT < P; j0 += kUnroll * NT) {
        double2 v[kUnroll];
#pragma unroll
        for (int i = 0; i < kUnroll; ++i) v[i] = part[first + j0 + (int64_t)i * NT];
#pragma unroll
        for (int i = 0; i < kUnroll; ++i)
            centred_add(S, Q, count(j0 + (int64_t)i * NT), v[i].x, v[i].y, R);
    }
    for (; j0 < P; j0 += NT) {
        const double2 v = part[first + j0];
        centred_add(S, Q, count(j0), v.x, v.y, R);
    }
    block_sum2<double, NT>(S, Q, lds);
    if (threadIdx.x == 0) {
        const double n = n_total;
        const double2 mm = centred_moments(S, Q, n, R);
        const double var = mm.y / n;
        const float hi = (float)mm.x;
        const float lo = (float)(mm.x - (double)hi);
        mean[u] = hi;
        rstd[u] = (float)(1.0 / sqrt(var + (double)eps));
        lo_ws[u] = lo;
        if (mean_lo) mean_lo[u] = lo;
    }
}

template <int NT = kThreads>
__device__ void finish_stats_unit(int64_t u, const double2* __restrict__ part,
                                  float* __restrict__ mean, float* __restrict__ rstd,
                                  float* __restrict__ mean_lo, float* __restrict__ lo_ws,
                                  int64_t HW, int64_t chunk, int64_t cpp, int64_t cpg,
                                  float eps, double* lds /*[2 * NT / 64]*/) {
    finish_unit<NT>(u, part, cpg * cpp, ChunkCount{HW, chunk, cpp}, (double)(cpg * HW), mean,
                    rstd, mean_lo, lo_ws, eps, lds);
}

// Finish of the depthwise forward's tile-group partials, one block per unit.
template <int NT>
__global__ __launch_bounds__(NT) void k_stats_finish_tiles(
    const double2* __restrict__ part, float* __restrict__ mean, float* __restrict__ rstd,
    float* __restrict__ mean_lo, float* __restrict__ lo_ws, int64_t P, TileCount count,
    double n_total, float eps) {
    __shared__ double lds[2 * NT / 64];
    finish_unit<NT>(blockIdx.x, part, P, count, n_total, mean, rstd, mean_lo, lo_ws, eps, lds);
}

// Finish-only grid for units of many chunk partials (a pointwise
// convolution's epilogue writes one per pixel chunk of each plane: 16384
// per unit at 4 x 2048^2): 1024 threads per unit instead of 256, so each
// thread combines a quarter as many.  At 64 -> 64 channels over 2048^2
// pixels, 16 units: 16.0 -> 8.4 us.
constexpr int kWideThreads = 1024;
constexpr int64_t kWideFinish = 8192;  // partials per unit from which it runs
__global__ __launch_bounds__(kWideThreads) void k_stats_finish_wide(
    const double2* __restrict__ part, float* __restrict__ mean, float* __restrict__ rstd,
    float* __restrict__ mean_lo, float* __restrict__ lo_ws, int64_t HW, int64_t chunk,
    int64_t cpp, int64_t cpg, int64_t fin_u0, float eps) {
    __shared__ double lds[2 * kWideThreads / 64];
    finish_stats_unit<kWideThreads>(fin_u0 + blockIdx.x, part, mean, rstd, mean_lo, lo_ws, HW,
                                    chunk, cpp, cpg, eps, lds);
}

// U: 128-bit loads in flight per thread.  The thread's first batch is
// issued whole before its shift K (the first element) is taken from it, so
// a chunk of 8 vectors per thread costs 8 / U memory round trips.  The
// elements reach each of the four accumulation lanes in index order for
// every U, so the partials do not depend on U.  NTL: chunk blocks b <
// nt_end use non-temporal loads (the rest, the tail that the reverse-walking
// second pass reads first, use cached loads, so it is still in the MALL).
template <bool VEC, int U, bool NTL>
__global__ __launch_bounds__(kThreads) void k_stats(
    const float* __restrict__ x, double2* __restrict__ part, float* __restrict__ mean,
    float* __restrict__ rstd, float* __restrict__ mean_lo, float* __restrict__ lo_ws,
    int64_t HW, int64_t chunk, int64_t cpp, int64_t cpg, int64_t fin_u0, int64_t fin_nu,
    int64_t block0, float eps, int64_t nt_end) {
    __shared__ double lds[4 * kWaves];
    if ((int64_t)blockIdx.x < fin_nu) {
        finish_stats_unit(fin_u0 + blockIdx.x, part, mean, rstd, mean_lo, lo_ws, HW, chunk,
                          cpp, cpg, eps, lds);
        return;
    }
    const int64_t b = chunk_block(block0, fin_nu);
    const Chunk ck = chunk_of(b, HW, chunk, cpp);
    const float* p = x + ck.plane * HW + ck.off;
    const int t = threadIdx.x;

    float K = 0.0f;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
    int64_t cnt = 0;
    if (VEC) {
        const f4* p4 = reinterpret_cast<const f4*>(p);
        const int64_t n4 = ck.len >> 2;
        auto walk = [&](auto ntl) {
        constexpr bool L = decltype(ntl)::value;
#define SOAR_ACC4(v)                                                     \
    {                                                                    \
        float d0 = (v).x - K, d1 = (v).y - K, d2 = (v).z - K,            \
              d3 = (v).w - K;                                            \
        s0 += d0; s1 += d1; s2 += d2; s3 += d3;                          \
        q0 = fmaf(d0, d0, q0); q1 = fmaf(d1, d1, q1);                    \
        q2 = fmaf(d2, d2, q2); q3 = fmaf(d3, d3, q3);                    \
    }
        int64_t i = t;
        if (i < n4) {
            cnt = 4 * ((n4 - 1 - i) / kThreads + 1);
            if (i + (U - 1) * kThreads < n4) {
                f4 v[U];
#pragma unroll
                for (int u = 0; u < U; ++u) v[u] = load4<L>(&p4[i + u * kThreads]);
                K = v[0].x;
#pragma unroll
                for (int u = 0; u < U; ++u) SOAR_ACC4(v[u]);
                i += U * kThreads;
            } else {
                const f4 v = load4<L>(&p4[i]);
                K = v.x;
                SOAR_ACC4(v);
                i += kThreads;
            }
        }
        for (; i + (U - 1) * kThreads < n4; i += U * kThreads) {
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = load4<L>(&p4[i + u * kThreads]);
#pragma unroll
            for (int u = 0; u < U; ++u) SOAR_ACC4(v[u]);
        }
        for (; i < n4; i += kThreads) {
            f4 a = load4<L>(&p4[i]);
            SOAR_ACC4(a);
        }
        };
        if (NTL && b < nt_end)
            walk(std::true_type{});
        else
            walk(std::false_type{});
#undef SOAR_ACC4
    } else {
        int64_t i = t;
        if (i < ck.len) {
            cnt = (ck.len - 1 - i) / kThreads + 1;
            K = p[i];
            i += kThreads;
        }
        for (; i + 3 * kThreads < ck.len; i += 4 * kThreads) {
            float d0 = p[i] - K, d1 = p[i + kThreads] - K,
                  d2 = p[i + 2 * kThreads] - K, d3 = p[i + 3 * kThreads] - K;
            s0 += d0; s1 += d1; s2 += d2; s3 += d3;
            q0 = fmaf(d0, d0, q0); q1 = fmaf(d1, d1, q1);
            q2 = fmaf(d2, d2, q2); q3 = fmaf(d3, d3, q3);
        }
        for (; i < ck.len; i += kThreads) {
            float d0 = p[i] - K;
            s0 += d0;
            q0 = fmaf(d0, d0, q0);
        }
    }
    // the block's (mean, M2) (gn_moments.hpp)
    const double2 m = block_moments<kThreads>(K, (s0 + s1) + (s2 + s3), (q0 + q1) + (q2 + q3),
                                              (int)cnt, lds);
    if (t == 0) part[b] = m;
}

// Per-block coefficients of plane `plane`: xhat = fma(x - mu, r, e) with
// mu the fp32 mean and e = -mean_lo * r.  (x - mu is exact whenever x is
// within a factor two of mu, Sterbenz.)
struct PlaneCoef {
    int64_t c, n, u;
    float mu, r, e, gm, bt;
};

__device__ __forceinline__ PlaneCoef plane_coef(
    int64_t plane, int64_t C, int64_t G, int64_t cpg,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ mean_lo) {
    PlaneCoef k;
    k.n = plane / C;
    k.c = plane - k.n * C;
    k.u = k.n * G + k.c / cpg;
    k.mu = mean[k.u];
    k.r = rstd[k.u];
    k.e = mean_lo ? -mean_lo[k.u] * k.r : 0.0f;
    k.gm = gamma ? gamma[k.c] : 1.0f;
    k.bt = beta ? beta[k.c] : 0.0f;
    return k;
}

// ======================================================================
// Folded finish for mid-size units (at most Tuning::fold_max partials per
// unit, one batch): instead of a finish launch between the passes, every
// second-pass block combines its own unit's partials before its work.
// All blocks of a unit run the same combine in the same order, so they
// agree bit for bit, and the statistics equal the separate finish's
// (finish_unit on kThreads threads): the block's thread t stands in for
// that finish's threads t, t + NT, ..., runs each one's partials in that
// one's order, and the wave sums are added in the same order.
// ======================================================================
constexpr int64_t kFoldMax = 4096;  // partials per unit

// Sum of (a, b) over an NT-thread block in a fixed order (wave trees, then
// the waves in order), returned to every thread.
template <int NT>
__device__ __forceinline__ double2 fold_block_sum2(double a, double b) {
    __shared__ double2 lds[NT / 64];
    a = wave_sum(a);
    b = wave_sum(b);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = make_double2(a, b);
    __syncthreads();
    double2 r = lds[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
        r.x += lds[i].x;
        r.y += lds[i].y;
    }
    __syncthreads();
    return r;
}

struct UnitStats {
    float hi, r, lo;
};

// Each virtual thread's partials j, j + kThreads, ... in batches of four
// loads issued together (indices clamped into the unit, the terms past P
// not added), so a unit of a few hundred partials costs one or two memory
// round trips.
template <int NT, typename Count>
__device__ UnitStats fold_unit_stats(int64_t u, const double2* __restrict__ part, int64_t P,
                                     const Count& count, double n_total, float eps) {
    constexpr int V = kThreads / NT;  // threads of the separate finish per thread
    constexpr int W = NT / 64;
    static_assert(V * NT == kThreads && W * 64 == NT, "block size");
    constexpr int kB = 4;
    __shared__ double2 sw[kThreads / 64];
    __shared__ float bc[3];
    const double2* __restrict__ pu = part + u * P;
    const double R = pu[0].x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int h = 0; h < V; ++h) {
        double S = 0.0, Q = 0.0;
        for (int64_t j0 = threadIdx.x + h * NT; j0 < P; j0 += kB * kThreads) {
            double2 v[kB];
#pragma unroll
            for (int i = 0; i < kB; ++i) v[i] = pu[min(j0 + (int64_t)i * kThreads, P - 1)];
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int64_t j = j0 + (int64_t)i * kThreads;
                if (j < P) centred_add(S, Q, count(j), v[i].x, v[i].y, R);
            }
        }
        S = wave_sum(S);
        Q = wave_sum(Q);
        if (lane == 0) sw[h * W + w] = make_double2(S, Q);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double S = sw[0].x, Q = sw[0].y;
#pragma unroll
        for (int i = 1; i < kThreads / 64; ++i) {
            S += sw[i].x;
            Q += sw[i].y;
        }
        const double2 mm = centred_moments(S, Q, n_total, R);
        const double var = mm.y / n_total;
        const float hi = (float)mm.x;
        bc[0] = hi;
        bc[1] = (float)(1.0 / sqrt(var + (double)eps));
        bc[2] = (float)(mm.x - (double)hi);
    }
    __syncthreads();
    return UnitStats{bc[0], bc[1], bc[2]};
}


// (S1, S2) of unit u from its backward partials: thread q adds gamma_j *
// partial q, q + NT, ..., j the partial's channel.
template <int NT>
__device__ double2 fold_unit_sums(int64_t u, const double2* __restrict__ part,
                                  const float* __restrict__ gamma, int64_t C, int64_t cpg,
                                  int64_t cpp) {
    const int64_t P = cpg * cpp;
    double a = 0.0, b = 0.0;
    for (int64_t q = threadIdx.x; q < P; q += NT) {
        const double2 v = part[u * P + q];
        const int64_t plane = u * cpg + q / cpp;
        const double g = gamma ? (double)gamma[plane % C] : 1.0;
        a += g * v.x;
        b += g * v.y;
    }
    return fold_block_sum2<NT>(a, b);
}

// dbeta[c] += sdz, dgamma[c] += sdzx; either output may be null (the
// reference guards each on its own, normalization_kernels.cu:142-152).
__device__ __forceinline__ void add_params(int64_t c, double sdz, double sdzx,
                                           float* __restrict__ dgamma,
                                           float* __restrict__ dbeta) {
    if (dbeta) dbeta[c] = (float)((double)dbeta[c] + sdz);
    if (dgamma) dgamma[c] = (float)((double)dgamma[c] + sdzx);
}

// dbeta[c] += sum over samples and chunks of channel c's sum(dz), dgamma[c]
// += the same of sum(dz * xhat) (the k_param_finish step, for one channel).
template <int NT>
__device__ void fold_param(int64_t c, const double2* __restrict__ part, int64_t N, int64_t C,
                           int64_t cpp, float* __restrict__ dgamma, float* __restrict__ dbeta) {
    double a = 0.0, b = 0.0;
    for (int64_t i = threadIdx.x; i < N * cpp; i += NT) {
        const int64_t n = i / cpp, q = i - n * cpp;
        const double2 v = part[(n * C + c) * cpp + q];
        a += v.x;
        b += v.y;
    }
    const double2 r = fold_block_sum2<NT>(a, b);
    if (threadIdx.x == 0) add_params(c, r.x, r.y, dgamma, dbeta);
}

// ======================================================================
// Forward pass 2: y = f((x - mean) * (gamma*rstd) + beta) [+ x].
// FOLD: the unit's statistics come from the partials (see above), chunk
// partials (kFoldChunks) or the depthwise forward's tile groups
// (kFoldTiles); the unit's first block also writes them out.
// ======================================================================
struct FoldArgs {
    const double2* part;  // chunk partials of the first pass
    float* mean;          // statistics out (forward)
    float* rstd;
    float* mean_lo;       // nullable
    float* dgamma;        // parameter gradients (backward), nullable
    float* dbeta;
    int64_t N, chunk, cpp;
    float eps;
    // backward without FOLD: the per-plane sums, non-null when the dx
    // launch also runs k_param_finish's sums (every plane sum is final)
    const double2* plane_sums;
    TileCount tiles;  // FOLD == kFoldTiles: the depthwise forward's tile groups
    const float* res;  // k_apply with XRES: the residual added instead of x
};

constexpr int kFoldChunks = 1, kFoldTiles = 2;

// XRES (with RES): the residual is fa.res, another tensor of x's shape,
// instead of x.
template <bool VEC, bool SILU, bool RES, bool NT, bool NTL, int FOLD, bool XRES = false>
__global__ __launch_bounds__(kThreads2) void k_apply(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ mean_lo,
    float* __restrict__ y, int64_t C, int64_t G, int64_t cpg, int64_t HW,
    int64_t chunk2, int64_t cpp2, int64_t block0, int64_t nb, int reverse, FoldArgs fa) {
    const int64_t b = batch_block(block0, nb, reverse);
    const Chunk ck = chunk_of(b, HW, chunk2, cpp2);
    PlaneCoef k;
    if (FOLD) {
        k.n = ck.plane / C;
        k.c = ck.plane - k.n * C;
        k.u = k.n * G + k.c / cpg;
        const double n = (double)(cpg * HW);
        UnitStats st;
        if constexpr (FOLD == kFoldTiles)
            st = fold_unit_stats<kThreads2>(k.u, fa.part, cpg * fa.tiles.tpp, fa.tiles, n,
                                            fa.eps);
        else
            st = fold_unit_stats<kThreads2>(k.u, fa.part, cpg * fa.cpp,
                                            ChunkCount{HW, fa.chunk, fa.cpp}, n, fa.eps);
        k.mu = st.hi;
        k.r = st.r;
        k.e = -st.lo * st.r;
        k.gm = gamma ? gamma[k.c] : 1.0f;
        k.bt = beta ? beta[k.c] : 0.0f;
        if (threadIdx.x == 0 && ck.plane % cpg == 0 && ck.off == 0) {
            fa.mean[k.u] = st.hi;
            fa.rstd[k.u] = st.r;
            if (fa.mean_lo) fa.mean_lo[k.u] = st.lo;
        }
    } else {
        k = plane_coef(ck.plane, C, G, cpg, gamma, beta, mean, rstd, mean_lo);
    }
    // z = gamma*xhat + beta = (x - mu)*(gamma*r) + (beta + gamma*e)
    const float a = k.gm * k.r, mu = k.mu, bt = fmaf(k.gm, k.e, k.bt);
    const int64_t base = ck.plane * HW + ck.off;
    const int t = threadIdx.x;
    // (the external residual is added to the rounded output, as an add
    // after the forward would: the empty asm keeps the add from contracting
    // with SiLU's last multiply)
    auto f = [&](float v, float rv) {
        float z = fmaf(v - mu, a, bt);
        float o = SILU ? silu_fast(z) : z;
        if constexpr (XRES) {
            asm volatile("" : "+v"(o));
            return o + rv;
        } else {
            return RES ? o + rv : o;
        }
    };
    if (VEC) {
        const f4* x4 = reinterpret_cast<const f4*>(x + base);
        const f4* r4 = reinterpret_cast<const f4*>((XRES ? fa.res : x) + base);
        f4* y4 = reinterpret_cast<f4*>(y + base);
        const int64_t n4 = ck.len >> 2;
        int64_t i = t;
        for (; i + (kLoads2 - 1) * kThreads2 < n4; i += kLoads2 * kThreads2) {
            f4 v[kLoads2], r[kLoads2];
#pragma unroll
            for (int u = 0; u < kLoads2; ++u) {
                v[u] = load4<NTL>(&x4[i + u * kThreads2]);
                if (XRES) r[u] = load4<NTL>(&r4[i + u * kThreads2]);
            }
#pragma unroll
            for (int u = 0; u < kLoads2; ++u) {
                const f4 rv = XRES ? r[u] : v[u];
                const f4 o = {f(v[u].x, rv.x), f(v[u].y, rv.y), f(v[u].z, rv.z),
                              f(v[u].w, rv.w)};
                store4<NT>(&y4[i + u * kThreads2], o);
            }
        }
        for (; i < n4; i += kThreads2) {
            const f4 v = load4<NTL>(&x4[i]);
            const f4 rv = XRES ? load4<NTL>(&r4[i]) : v;
            f4 o = {f(v.x, rv.x), f(v.y, rv.y), f(v.z, rv.z), f(v.w, rv.w)};
            store4<NT>(&y4[i], o);
        }
    } else {
        const float* xp = x + base;
        const float* rp = (XRES ? fa.res : x) + base;
        float* yp = y + base;
        for (int64_t i = t; i < ck.len; i += kThreads2) store1<NT>(&yp[i], f(xp[i], rp[i]));
    }
}

// ======================================================================
// Backward pass 1: finish of the previous batch's units, then per-chunk
// sum(dz) and sum(dz * xhat) of this batch, dz the gradient at the
// GroupNorm output (SiLU derivative recomputed from x).
// A finish block sums each plane of its unit over the plane's chunks
// (plane_sums, float64, fixed order) and forms
//   S1 = sum_c gamma_c * sum dz,   S2 = sum_c gamma_c * sum dz*xhat.
// The block's lanes form groups of gs = min(64, cpp rounded up to a power
// of two) lanes, one plane per group at a time (group g takes planes
// g, g + ngroups, ...), so the planes' loads are in flight together
// instead of one plane after another; each group adds its planes'
// weighted sums in plane order and thread 0 adds the groups in order.
//
// Mean residual recovery (part_x non-null: no SiLU and no saved mean_lo,
// as behind the reference-signature group_norm_backward, whose forward
// saves the fp32 mean alone).  The chunks then hold sum(dy * xhat32) with
// xhat32 = (x - mu32) * r, and part_x the chunk sums of x - mu32.  Their
// unit sum over M is lo = mean - mu32, so the true xhat is xhat32 + e with
// e = -lo * r; since dz = dy does not depend on xhat,
//   sum dz * xhat = sum dz * xhat32 + e * sum dz
// corrects every plane exactly.  lo goes to lo_ws for the dx pass.
// ======================================================================
__device__ void finish_bwd_unit(int64_t u, const double2* __restrict__ part,
                                const double* __restrict__ part_x,
                                const float* __restrict__ gamma,
                                const float* __restrict__ rstd, float* __restrict__ lo_ws,
                                double2* __restrict__ plane_sums,
                                double2* __restrict__ unit_sums, int64_t C, int64_t HW,
                                int64_t cpp, int64_t cpg, double* lds /*[2 * kThreads]*/) {
    double e = 0.0;
    if (part_x) {
        const int64_t P = cpg * cpp;
        double sx = 0.0;
        for (int64_t q = threadIdx.x; q < P; q += kThreads) sx += part_x[u * P + q];
        sx = wave_sum(sx);
        if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = sx;
        __syncthreads();
        sx = lds[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) sx += lds[i];
        __syncthreads();
        const float lo = (float)(sx / (double)(cpg * HW));
        e = (double)(-lo * rstd[u]);  // the dx pass's e, in its fp32 form
        if (threadIdx.x == 0) lo_ws[u] = lo;
    }
    static_assert(kThreads == kBwdFinishThreads, "bwd_unit_sums follows this block's order");
    const int gs = bwd_plane_lanes((int)cpp);  // cpp < 2^31 (the reduction's grid)
    const int ngroups = kThreads / gs;
    const int grp = (int)threadIdx.x / gs, r = (int)threadIdx.x & (gs - 1);
    double S1 = 0.0, S2 = 0.0;  // meaningful in each group's lane r == 0
    for (int64_t j = grp; j - grp < cpg; j += ngroups) {
        const bool live = j < cpg;
        const int64_t plane = u * cpg + (live ? j : 0);
        const double2 ab = bwd_plane_sum(part + plane * cpp, (int)cpp, gs, r, live);
        double A = ab.x, B = ab.y;
        if (live && r == 0) {
            B = fma(e, A, B);
            plane_sums[plane] = make_double2(A, B);
            const double gj = gamma ? (double)gamma[plane % C] : 1.0;
            S1 += gj * A;
            S2 += gj * B;
        }
    }
    if (r == 0) {
        lds[grp] = S1;
        lds[kThreads + grp] = S2;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s1 = 0.0, s2 = 0.0;
        for (int g = 0; g < ngroups; ++g) {
            s1 += lds[g];
            s2 += lds[kThreads + g];
        }
        unit_sums[u] = make_double2(s1, s2);
    }
}

// LOREC: mean residual recovery (see finish_bwd_unit); also writes the
// chunk sums of x - mu to part_x.  Only without SiLU, so dz = dy.
// U: 128-bit loads in flight per thread, U/2 of each tensor (elements reach
// each accumulation lane in index order for every U).  NTL: chunk blocks
// b < nt_end use non-temporal loads (as in k_stats).
template <bool VEC, bool SILU, bool LOREC, int U, bool NTL>
__global__ __launch_bounds__(kThreads) void k_bwd_reduce(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ mean_lo, double2* __restrict__ part,
    double* __restrict__ part_x, float* __restrict__ lo_ws,
    double2* __restrict__ plane_sums, double2* __restrict__ unit_sums, int64_t C, int64_t G,
    int64_t cpg, int64_t HW, int64_t chunk, int64_t cpp, int64_t fin_u0, int64_t fin_nu,
    int64_t block0, int64_t nt_end) {
    static_assert(!(SILU && LOREC), "the mean residual is recovered only when dz = dy");
    __shared__ float lds[2 * kWaves];
    __shared__ double ldsd[2 * kThreads];
    if ((int64_t)blockIdx.x < fin_nu) {
        finish_bwd_unit(fin_u0 + blockIdx.x, part, LOREC ? part_x : nullptr, gamma, rstd,
                        lo_ws, plane_sums, unit_sums, C, HW, cpp, cpg, ldsd);
        return;
    }
    const int64_t b = chunk_block(block0, fin_nu);
    const Chunk ck = chunk_of(b, HW, chunk, cpp);
    const PlaneCoef k = plane_coef(ck.plane, C, G, cpg, gamma, beta, mean, rstd,
                                   LOREC ? nullptr : mean_lo);
    const float mu = k.mu, r = k.r, e = k.e, gm = k.gm, bt = k.bt;
    const int64_t base = ck.plane * HW + ck.off;
    const int t = threadIdx.x;
    float sa0 = 0.f, sa1 = 0.f, sb0 = 0.f, sb1 = 0.f, sc0 = 0.f, sc1 = 0.f;
    auto acc = [&](float g, float v, float& sa, float& sb, float& sc) {
        const float d = v - mu;
        float xh = fmaf(d, r, e);
        float dz = SILU ? dsilu_fast(g, fmaf(gm, xh, bt)) : g;
        sa += dz;
        sb = fmaf(dz, xh, sb);
        if (LOREC) sc += d;
    };
    if (VEC) {
        const f4* x4 = reinterpret_cast<const f4*>(x + base);
        const f4* g4 = reinterpret_cast<const f4*>(dy + base);
        const int64_t n4 = ck.len >> 2;
        constexpr int UH = U / 2;
        auto walk = [&](auto ntl) {
        constexpr bool L = decltype(ntl)::value;
        int64_t i = t;
        for (; i + (UH - 1) * kThreads < n4; i += UH * kThreads) {
            f4 v[UH], g[UH];
#pragma unroll
            for (int u = 0; u < UH; ++u) {
                v[u] = load4<L>(&x4[i + u * kThreads]);
                g[u] = load4<L>(&g4[i + u * kThreads]);
            }
#pragma unroll
            for (int u = 0; u < UH; ++u) {
                acc(g[u].x, v[u].x, sa0, sb0, sc0); acc(g[u].y, v[u].y, sa1, sb1, sc1);
                acc(g[u].z, v[u].z, sa0, sb0, sc0); acc(g[u].w, v[u].w, sa1, sb1, sc1);
            }
        }
        for (; i < n4; i += kThreads) {
            f4 v0 = load4<L>(&x4[i]), g0 = load4<L>(&g4[i]);
            acc(g0.x, v0.x, sa0, sb0, sc0); acc(g0.y, v0.y, sa1, sb1, sc1);
            acc(g0.z, v0.z, sa0, sb0, sc0); acc(g0.w, v0.w, sa1, sb1, sc1);
        }
        };
        if (NTL && b < nt_end)
            walk(std::true_type{});
        else
            walk(std::false_type{});
    } else {
        const float* xp = x + base;
        const float* gp = dy + base;
        for (int64_t i = t; i < ck.len; i += kThreads) acc(gp[i], xp[i], sa0, sb0, sc0);
    }
    float sa = sa0 + sa1, sb = sb0 + sb1;
    if (LOREC) {
        // the chunk's sum of x - mu first (its own exchange: block_sum2
        // below ends with the block synchronised before lds is reused)
        float sc = sc0 + sc1, dummy = 0.0f;
        block_sum2(sc, dummy, lds);
        if (t == 0) part_x[b] = (double)sc;
    }
    block_sum2(sa, sb, lds);
    if (t == 0) part[b] = make_double2((double)sa, (double)sb);
}

// dgamma[c] += sum_n sum dz*xhat, dbeta[c] += sum_n sum dz, in sample
// order (the reference accumulates parameter gradients per sample,
// tensor.cpp:173-192).
__global__ void k_param_finish(const double2* __restrict__ plane_sums,
                               float* __restrict__ dgamma, float* __restrict__ dbeta,
                               int64_t N, int64_t C) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    double a = 0.0, b = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        const double2 v = plane_sums[n * C + c];
        a += v.x;
        b += v.y;
    }
    add_params(c, a, b, dgamma, dbeta);
}

// ======================================================================
// Backward pass 2: dx = A*dz + D*xhat + B [+ dy] [+ dx_old] with
// A = gamma_c*rstd, B = -rstd*S1/M, D = -rstd*S2/M.
// ======================================================================
// FOLD: S1 / S2 come from the unit's chunk partials, and the block of
// channel c's first chunk in sample 0 also adds channel c's dgamma / dbeta
// (the folded k_param_finish).
template <bool VEC, bool SILU, bool RES, bool ACC, bool NT, bool NTL, bool FOLD>
__global__ __launch_bounds__(kThreadsDx) void k_bwd_dx(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ mean_lo, const double2* __restrict__ unit_sums,
    float* __restrict__ dx, int64_t C, int64_t G, int64_t cpg, int64_t HW,
    int64_t chunk2, int64_t cpp2, int64_t block0, int64_t nb, int reverse, FoldArgs fa) {
    const int64_t b = batch_block(block0, nb, reverse);
    const Chunk ck = chunk_of(b, HW, chunk2, cpp2);
    const PlaneCoef k = plane_coef(ck.plane, C, G, cpg, gamma, beta, mean, rstd, mean_lo);
    double2 S;
    if (FOLD) {
        S = fold_unit_sums<kThreadsDx>(k.u, fa.part, gamma, C, cpg, fa.cpp);
        if ((fa.dgamma || fa.dbeta) && k.n == 0 && ck.off == 0)
            fold_param<kThreadsDx>(k.c, fa.part, fa.N, C, fa.cpp, fa.dgamma, fa.dbeta);
    } else {
        S = unit_sums[k.u];
        if (fa.plane_sums && k.n == 0 && ck.off == 0 && threadIdx.x == 0) {
            // k_param_finish for channel c, same sums in the same order
            double sa = 0.0, sb = 0.0;
            for (int64_t n = 0; n < fa.N; ++n) {
                const double2 v = fa.plane_sums[n * C + k.c];
                sa += v.x;
                sb += v.y;
            }
            add_params(k.c, sa, sb, fa.dgamma, fa.dbeta);
        }
    }
    const double Md = (double)(cpg * HW);
    const float mu = k.mu, r = k.r, e = k.e, gm = k.gm, bt = k.bt;
    const float A = gm * r;
    const float B = (float)(-(double)r * S.x / Md);
    const float D = (float)(-(double)r * S.y / Md);
    const int64_t base = ck.plane * HW + ck.off;
    const int t = threadIdx.x;
    auto f = [&](float g, float v, float old) {
        float xh = fmaf(v - mu, r, e);
        float dz = SILU ? dsilu_fast(g, fmaf(gm, xh, bt)) : g;
        float o = fmaf(A, dz, fmaf(D, xh, B));
        if (RES) o += g;
        if (ACC) o += old;
        return o;
    };
    if (VEC) {
        const f4* x4 = reinterpret_cast<const f4*>(x + base);
        const f4* g4 = reinterpret_cast<const f4*>(dy + base);
        f4* o4 = reinterpret_cast<f4*>(dx + base);
        const int64_t n4 = ck.len >> 2;
        int64_t i = t;
        for (; i + (kLoadsDx - 1) * kThreadsDx < n4; i += kLoadsDx * kThreadsDx) {
            f4 v[kLoadsDx], g[kLoadsDx], p[kLoadsDx];
#pragma unroll
            for (int u = 0; u < kLoadsDx; ++u) {
                v[u] = load4<NTL>(&x4[i + u * kThreadsDx]);
                g[u] = load4<NTL>(&g4[i + u * kThreadsDx]);
                p[u] = ACC ? o4[i + u * kThreadsDx] : f4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < kLoadsDx; ++u) {
                const f4 r = {f(g[u].x, v[u].x, p[u].x), f(g[u].y, v[u].y, p[u].y),
                              f(g[u].z, v[u].z, p[u].z), f(g[u].w, v[u].w, p[u].w)};
                store4<NT>(&o4[i + u * kThreadsDx], r);
            }
        }
        for (; i < n4; i += kThreadsDx) {
            f4 v0 = load4<NTL>(&x4[i]), g0 = load4<NTL>(&g4[i]);
            f4 p0 = {0.f, 0.f, 0.f, 0.f};
            if (ACC) p0 = o4[i];
            f4 r0 = {f(g0.x, v0.x, p0.x), f(g0.y, v0.y, p0.y),
                     f(g0.z, v0.z, p0.z), f(g0.w, v0.w, p0.w)};
            store4<NT>(&o4[i], r0);
        }
    } else {
        const float* xp = x + base;
        const float* gp = dy + base;
        float* op = dx + base;
        for (int64_t i = t; i < ck.len; i += kThreadsDx)
            store1<NT>(&op[i], f(gp[i], xp[i], ACC ? op[i] : 0.0f));
    }
}

// ======================================================================
// Small units: the whole layer in one launch per direction.  The SOAR
// model's GroupNorms at small images are a few thousand elements per unit;
// there the multi-kernel path is dominated by its launches.
//
// One 1024-thread block owns a unit (forward) or a group across samples
// (backward).  Channel j of the unit goes to tpc = 1024 / cpgp consecutive
// threads (cpgp = cpg rounded up to a power of two), each holding up to 32
// of the channel's HW elements in registers: x (and dy) are read once and
// y (dx) written once.  Per-channel sums reduce over the tpc threads of a
// channel with shuffles (and LDS across waves when tpc > 64), whole-unit
// sums over the block, always in a fixed order.
//
// Forward statistics are float64 sums of x - K (K = the unit's first
// element) and of its square; the apply is k_apply's (fp32 mean, its
// rounding residual folded into the shift).
// ======================================================================
// Block sizes: NT = 256 for units of at most 256 * 32 elements, else 1024.
constexpr int kSmallThreads = 1024;
constexpr int kSmallPer = 32;  // elements per thread
constexpr int kSmallHalf = 16;  // elements per load batch of the backward
constexpr int kMaxSmallCpg = 256;  // channels per group (>= 4 threads each)

struct SmallMap {
    int tpc;   // threads per channel (power of two, >= 4)
    int j, r;  // this thread's channel and its rank in the channel
    int nk;    // this thread's elements: r + k*tpc for k < nk (0 if j >= cpg)
};

// (32-bit indices: a channel holds at most kSmallPer * 1024 elements)
__device__ __forceinline__ SmallMap small_map(int lg, int64_t cpg, int64_t HW) {
    SmallMap m;
    m.tpc = 1 << lg;
    m.j = (int)threadIdx.x >> lg;
    m.r = (int)threadIdx.x & (m.tpc - 1);
    m.nk = m.j < cpg ? ((int)HW - m.r + m.tpc - 1) >> lg : 0;
    return m;
}

// Loads this thread's elements of a unit through a raw buffer descriptor on
// the unit (wave-uniform base, 32-bit lane offsets: no 64-bit address per
// element).  The element step goes in the vector offset with the lane term,
// since the descriptor's range check covers the vector offset only: elements
// past the unit read 0 without touching memory; lanes past their channel
// read the next channel's values, which the callers never use (they test
// k < m.nk).
constexpr int kSmallRsrcWord3 = 0x00020000;  // gfx9-family raw buffer descriptor

template <int NV = kSmallPer>
__device__ __forceinline__ void small_load(const float* unit, int64_t M, int64_t HW,
                                           const SmallMap& m, float (&v)[NV], int k0 = 0) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(unit), (short)0,
                                                      (int)(M * 4), kSmallRsrcWord3);
    int vo = (m.j * (int)HW + m.r) * 4;
    asm volatile("" : "+v"(vo));  // each call loads anew (no reuse across calls)
#pragma unroll
    for (int k = 0; k < NV; ++k)
        v[k] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rs, vo + (k0 + k) * m.tpc * 4, 0, 0));
}

// Sums of (a, b) over the tpc threads of each channel; valid in the
// channel's rank-0 thread (xor tree within 64 lanes, else wave trees and
// then the channel's waves in order through LDS).
__device__ __forceinline__ void channel_sum2(double& a, double& b, const SmallMap& m,
                                             double2* lds) {
    if (m.tpc <= 64) {
        for (int off = m.tpc >> 1; off > 0; off >>= 1) {
            a += __shfl_xor(a, off);
            b += __shfl_xor(b, off);
        }
        return;
    }
    a = wave_sum(a);
    b = wave_sum(b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) lds[w] = make_double2(a, b);
    __syncthreads();
    double ra = 0.0, rb = 0.0;
    if (m.r == 0) {
        const int nw = m.tpc >> 6;
        for (int i = 0; i < nw; ++i) {
            ra += lds[w + i].x;
            rb += lds[w + i].y;
        }
    }
    __syncthreads();
    a = ra;
    b = rb;
}

template <bool SILU, bool RES>
__device__ __forceinline__ void small_apply_regs(const float (&xv)[kSmallPer], float* __restrict__ yc,
                                                 const SmallMap& m, float gm, float bt, float mu,
                                                 float r, float lo) {
    const float a = gm * r;
    const float b = fmaf(gm, -lo * r, bt);
#pragma unroll
    for (int k = 0; k < kSmallPer; ++k) {
        if (k < m.nk) {
            const float z = fmaf(xv[k] - mu, a, b);
            float o = SILU ? silu_fast(z) : z;
            if (RES) o += xv[k];
            yc[m.r + k * m.tpc] = o;
        }
    }
}

template <int NT, bool SILU, bool RES>
__global__ __launch_bounds__(NT) void k_small_fwd(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ y, float* __restrict__ mean,
    float* __restrict__ rstd, float* __restrict__ mean_lo, int64_t G, int64_t cpg, int64_t HW,
    int lg, float eps) {
    __shared__ double2 lds[NT / 64];
    const int64_t u = blockIdx.x;
    const SmallMap m = small_map(lg, cpg, HW);
    const bool live = m.j < cpg;
    // the affine parameters' loads go out with the unit's
    const int64_t c = (u % G) * cpg + m.j;
    const float gm = (live && gamma) ? gamma[c] : 1.0f;
    const float bt = (live && beta) ? beta[c] : 0.0f;
    float xv[kSmallPer];
    small_load(x + u * cpg * HW, cpg * HW, HW, m, xv);  // a unit is contiguous in NCHW
    const double K = (double)x[u * cpg * HW];
    double s = 0.0, q = 0.0;
#pragma unroll
    for (int k = 0; k < kSmallPer; ++k) {
        if (k < m.nk) {
            const double d = (double)xv[k] - K;
            s += d;
            q = fma(d, d, q);
        }
    }
    // both sums over the block in one exchange, waves added in order
    s = wave_sum(s);
    q = wave_sum(q);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = make_double2(s, q);
    __syncthreads();
    s = lds[0].x;
    q = lds[0].y;
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
        s += lds[i].x;
        q += lds[i].y;
    }
    const double M = (double)(cpg * HW);
    const double sm = s / M;
    const double md = K + sm;
    const double var = fmax(q / M - sm * sm, 0.0);
    const float hi = (float)md;
    const float lo = (float)(md - (double)hi);
    const float r = (float)(1.0 / sqrt(var + (double)eps));
    if (threadIdx.x == 0) {
        mean[u] = hi;
        rstd[u] = r;
        if (mean_lo) mean_lo[u] = lo;
    }
    small_apply_regs<SILU, RES>(xv, y + (u * cpg + (live ? m.j : 0)) * HW, m, gm, bt, hi, r, lo);
}

// The GroupNorm after a pointwise convolution whose epilogue wrote the
// chunk partials: the unit's finish (its cpg*cpp partials, combined in a
// fixed order), then its apply, in one block.
template <int NT, bool SILU, bool RES>
__global__ __launch_bounds__(NT) void k_small_finish_apply(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ y, const double2* __restrict__ part,
    float* __restrict__ mean, float* __restrict__ rstd, float* __restrict__ mean_lo,
    float* __restrict__ lo_ws, int64_t G, int64_t cpg, int64_t HW, int64_t chunk, int64_t cpp,
    int lg, float eps) {
    __shared__ double2 ldsq[NT / 64];
    __shared__ float bc[3];
    const int64_t u = blockIdx.x;
    const SmallMap m = small_map(lg, cpg, HW);
    const bool live = m.j < cpg;
    float xv[kSmallPer];  // loads in flight while the partials combine
    small_load(x + u * cpg * HW, cpg * HW, HW, m, xv);
    const int64_t P = cpg * cpp;
    // sums about partial 0's mean (centred_add), threads then waves in order
    const double R = part[u * P].x;
    double S = 0.0, Q = 0.0;
    for (int64_t q = threadIdx.x; q < P; q += NT) {
        const double2 v = part[u * P + q];
        centred_add(S, Q, partial_count(q, HW, chunk, cpp), v.x, v.y, R);
    }
    S = wave_sum(S);
    Q = wave_sum(Q);
    if ((threadIdx.x & 63) == 0) ldsq[threadIdx.x >> 6] = make_double2(S, Q);
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int i = 1; i < NT / 64; ++i) {
            S += ldsq[i].x;
            Q += ldsq[i].y;
        }
        const double n = (double)(cpg * HW);
        const double2 mm = centred_moments(S, Q, n, R);
        const double var = mm.y / n;
        const float hi = (float)mm.x;
        const float lo = (float)(mm.x - (double)hi);
        const float r = (float)(1.0 / sqrt(var + (double)eps));
        mean[u] = hi;
        rstd[u] = r;
        lo_ws[u] = lo;
        if (mean_lo) mean_lo[u] = lo;
        bc[0] = hi;
        bc[1] = r;
        bc[2] = lo;
    }
    __syncthreads();
    const int64_t c = (u % G) * cpg + m.j;
    const float gm = (live && gamma) ? gamma[c] : 1.0f;
    const float bt = (live && beta) ? beta[c] : 0.0f;
    small_apply_regs<SILU, RES>(xv, y + (u * cpg + (live ? m.j : 0)) * HW, m, gm, bt, bc[0],
                                bc[1], bc[2]);
}

// Backward: one block per group g walks the samples in order.  Per unit:
// per-channel float64 sums of dz and dz*xhat, S1 = sum_j gamma_j sum(dz)_j
// and S2 likewise (every wave forms them from LDS in the same fixed order,
// so no broadcast is needed), then dx.  ONE: a thread holds at most 16
// elements, kept in registers for dx; otherwise the elements come in two
// halves of 16 and dx reloads them (L2-resident): keeping both halves
// alive across the reductions would not fit in 128 registers.  The channel
// sums are added over samples in order into dgamma / dbeta at the end (as
// k_param_finish).  lorec (no SiLU, no saved mean_lo): the unit's mean
// residual is recovered from its sum of x - mu, as in finish_bwd_unit.
template <int NT, bool SILU, bool RES, bool ACC, bool ONE>
__global__ __launch_bounds__(NT) void k_small_bwd(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ mean_lo, float* __restrict__ dx,
    float* __restrict__ dgamma, float* __restrict__ dbeta, int64_t N, int64_t C, int64_t G,
    int64_t cpg, int64_t HW, int lg, int lorec) {
    constexpr int kHalves = ONE ? 1 : kSmallPer / kSmallHalf;
    __shared__ double chA[kMaxSmallCpg], chB[kMaxSmallCpg];
    __shared__ double2 lds[NT / 64];
    __shared__ double ldx[NT / 64];
    const int64_t g = blockIdx.x;
    const SmallMap m = small_map(lg, cpg, HW);
    const bool live = m.j < cpg;
    const int lane = threadIdx.x & 63;
    const int64_t c = g * cpg + m.j;
    const float gm = (live && gamma) ? gamma[c] : 1.0f;
    const float bt = (live && beta) ? beta[c] : 0.0f;
    double accA = 0.0, accB = 0.0;  // rank-0 thread of each channel: sums over samples
    for (int64_t n = 0; n < N; ++n) {
        const int64_t u = n * G + g;
        const int64_t off = (u * cpg + (live ? m.j : 0)) * HW;
        const float* xu = x + u * cpg * HW;
        const float* gu = dy + u * cpg * HW;
        const float mu = mean[u], r = rstd[u];
        float e = mean_lo ? -mean_lo[u] * r : 0.0f;
        double sa = 0.0, sb = 0.0, sx = 0.0;
        float xv[kSmallHalf], gv[kSmallHalf];
#pragma unroll
        for (int hh = 0; hh < kHalves; ++hh) {
            const int h = hh * kSmallHalf;
            small_load<kSmallHalf>(xu, cpg * HW, HW, m, xv, h);
            small_load<kSmallHalf>(gu, cpg * HW, HW, m, gv, h);
#pragma unroll
            for (int k = 0; k < kSmallHalf; ++k) {
                if (h + k < m.nk) {
                    const float xh = fmaf(xv[k] - mu, r, e);
                    const float dz = SILU ? dsilu_fast(gv[k], fmaf(gm, xh, bt)) : gv[k];
                    sa += (double)dz;
                    sb = fma((double)dz, (double)xh, sb);
                    if (lorec) sx += (double)(xv[k] - mu);
                }
            }
        }
        channel_sum2(sa, sb, m, lds);
        if (lorec) {
            // whole-unit sum of x - mu (waves in order) -> lo, e; the
            // channel sums were formed with e = 0 and dz = dy
            double tx = wave_sum(sx);
            if (lane == 0) ldx[threadIdx.x >> 6] = tx;
            __syncthreads();
            tx = ldx[0];
#pragma unroll
            for (int i = 1; i < NT / 64; ++i) tx += ldx[i];
            const float lo = (float)(tx / (double)(cpg * HW));
            e = -lo * r;
            sb = fma((double)e, sa, sb);
        }
        if (live && m.r == 0) {
            chA[m.j] = (double)gm * sa;
            chB[m.j] = (double)gm * sb;
            accA += sa;
            accB += sb;
        }
        __syncthreads();
        if (dx) {
            double s1 = 0.0, s2 = 0.0;
            for (int64_t j = lane; j < cpg; j += 64) {
                s1 += chA[j];
                s2 += chB[j];
            }
            s1 = __shfl(wave_sum(s1), 0);
            s2 = __shfl(wave_sum(s2), 0);
            const double Md = (double)(cpg * HW);
            const float B = (float)(-(double)r * s1 / Md);
            const float D = (float)(-(double)r * s2 / Md);
            float* dc = dx + off;
            if (ONE) {
                const float A = gm * r;
#pragma unroll
                for (int k = 0; k < kSmallHalf; ++k) {
                    const int i = m.r + k * m.tpc;
                    if (k < m.nk) {
                        const float xh = fmaf(xv[k] - mu, r, e);
                        const float dz = SILU ? dsilu_fast(gv[k], fmaf(gm, xh, bt)) : gv[k];
                        float o = fmaf(A, dz, fmaf(D, xh, B));
                        if (RES) o += gv[k];
                        if (ACC) o += dc[i];
                        dc[i] = o;
                    }
                }
            } else {
                float mu2 = mu, r2 = r, e2 = e, gm2 = gm, bt2 = bt;
                asm volatile("" : "+v"(mu2), "+v"(r2), "+v"(e2), "+v"(gm2), "+v"(bt2));
                const float A = gm2 * r2;
#pragma unroll
                for (int h = 0; h < kSmallPer; h += kSmallHalf) {
                    small_load<kSmallHalf>(xu, cpg * HW, HW, m, xv, h);
                    small_load<kSmallHalf>(gu, cpg * HW, HW, m, gv, h);
#pragma unroll
                    for (int k = 0; k < kSmallHalf; ++k) {
                        const int i = m.r + (h + k) * m.tpc;
                        if (h + k < m.nk) {
                            const float xh = fmaf(xv[k] - mu2, r2, e2);
                            const float dz =
                                SILU ? dsilu_fast(gv[k], fmaf(gm2, xh, bt2)) : gv[k];
                            float o = fmaf(A, dz, fmaf(D, xh, B));
                            if (RES) o += gv[k];
                            if (ACC) o += dc[i];
                            dc[i] = o;
                        }
                    }
                }
            }
        }
        if (n + 1 < N) __syncthreads();  // chA / chB are rewritten by the next sample
    }
    if ((dgamma || dbeta) && live && m.r == 0) add_params(c, accA, accB, dgamma, dbeta);
}

// ---- host-side dispatch over the template flags -------------------------

struct WsView {
    double2* part;        // [blocks]
    double2* plane_sums;  // [planes]
    double2* unit_sums;   // [units]
    float* lo;            // [units]
    double* part_x;       // [blocks] chunk sums of x - mu (mean residual recovery)
};

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

WsView ws_view(const Plan& p, void* ws) {
    char* c = static_cast<char*>(ws);
    WsView v;
    v.part = reinterpret_cast<double2*>(c);
    c += align256(sizeof(double2) * (size_t)p.blocks);
    v.plane_sums = reinterpret_cast<double2*>(c);
    c += align256(sizeof(double2) * (size_t)p.planes);
    v.unit_sums = reinterpret_cast<double2*>(c);
    c += align256(sizeof(double2) * (size_t)p.units);
    v.lo = reinterpret_cast<float*>(c);
    c += align256(sizeof(float) * (size_t)p.units);
    v.part_x = reinterpret_cast<double*>(c);
    return v;
}

// Calls f(std::integral_constant<int, U>) for U = 8 or 4 loads in flight.
template <typename F>
void loads_sel(int loads, F&& f) {
    if (loads == 8)
        f(std::integral_constant<int, 8>{});
    else
        f(std::integral_constant<int, 4>{});
}

// Calls f(std::true_type) or f(std::false_type): turns a runtime flag into
// a template argument.
template <typename F>
void bsel(bool b, F&& f) {
    if (b)
        f(std::true_type{});
    else
        f(std::false_type{});
}

// fold: the statistics come from partials (see fold_unit_stats) and are
// written out by the kernel: kFoldChunks, the chunk partials in the
// workspace; kFoldTiles, the depthwise forward's tile groups at `tpart`.
void launch_apply(const Plan& p, const Tuning& t, const FwdArgs& a, const float* lo,
                  int64_t block0, int64_t nb, hipStream_t s, int fold = 0,
                  const double2* tpart = nullptr, const TileCount& tiles = TileCount{}) {
    const bool silu = (a.flags & SOAR_GN_SILU) != 0;
    const bool res = (a.flags & SOAR_GN_RESIDUAL) != 0;
    const dim3 grid((unsigned)nb);
    const FoldArgs fa{fold == kFoldTiles ? tpart : ws_view(p, a.ws).part,
                      a.mean, a.rstd, a.mean_lo, nullptr, nullptr, p.N, p.chunk, p.cpp, a.eps,
                      nullptr, tiles, a.res};
    // an external residual (the SOAR LKR block's x + CBA(...))
    const bool xres = res && a.res != nullptr;
    auto go = [&](auto F) {
        bsel(p.vec4, [&](auto V) {
            bsel(t.nt_store != 0, [&](auto N) {
                bsel(V() && (t.nt_load & 1) != 0, [&](auto L) {
                    auto launch = [&](auto S, auto R, auto X) {
                        k_apply<V(), S(), R(), N(), L(), F(), X()><<<grid, kThreads2, 0, s>>>(
                            a.x, a.gamma, a.beta, a.mean, a.rstd, lo, a.y, p.C, p.G, p.cpg,
                            p.HW, p.chunk2, p.cpp2, block0, nb, t.reverse, fa);
                    };
                    if (xres) {
                        bsel(silu, [&](auto S) {
                            launch(S, std::true_type{}, std::true_type{});
                        });
                        return;
                    }
                    bsel(silu, [&](auto S) {
                        bsel(res, [&](auto R) { launch(S, R, std::false_type{}); });
                    });
                });
            });
        });
    };
    if (fold == kFoldTiles)
        go(std::integral_constant<int, kFoldTiles>{});
    else if (fold == kFoldChunks)
        go(std::integral_constant<int, kFoldChunks>{});
    else
        go(std::integral_constant<int, 0>{});
}

// fold: S1 / S2 and dgamma / dbeta come from the partials in the workspace.
void launch_dx(const Plan& p, const Tuning& t, const BwdArgs& a, const double2* unit_sums,
               int64_t block0, int64_t nb, hipStream_t s, bool fold = false,
               const double2* param_sums = nullptr) {
    const bool silu = (a.flags & SOAR_GN_SILU) != 0;
    const bool res = (a.flags & SOAR_GN_RESIDUAL) != 0;
    const bool accum = (a.flags & SOAR_GN_ACCUMULATE_DX) != 0;
    const dim3 grid((unsigned)nb);
    const FoldArgs fa{ws_view(p, a.ws).part, nullptr, nullptr, nullptr, a.dgamma, a.dbeta,
                      p.N, p.chunk, p.cpp, 0.0f, fold ? nullptr : param_sums};
    bsel(p.vec4, [&](auto V) {
        bsel(silu, [&](auto S) {
            bsel(res, [&](auto R) {
                bsel(accum, [&](auto A) {
                    bsel(t.nt_store != 0 && !accum, [&](auto N) {
                        bsel(V() && (t.nt_load & 1) != 0, [&](auto L) {
                            bsel(fold, [&](auto F) {
                                k_bwd_dx<V(), S(), R(), A(), N(), L(), F()>
                                    <<<grid, kThreadsDx, 0, s>>>(
                                        a.dy, a.x, a.gamma, a.beta, a.mean, a.rstd, a.mean_lo,
                                        unit_sums, a.dx, p.C, p.G, p.cpg, p.HW, p.chunk2,
                                        p.cpp2, block0, nb, t.reverse, fa);
                            });
                        });
                    });
                });
            });
        });
    });
}

// Mid-size units fold the finish into the second pass: one batch, at most
// t.fold_max (<= kFoldMax) partials per unit, and more than kFoldAlways
// only for units of at most kFoldBigUnit elements.  Every second-pass block
// re-reads its unit's partials (16 bytes each, from L2): next to a 4096-
// float chunk that is cheap up to a hundred or so, and past that it pays
// only where the unit's blocks are few and the saved launch is a large
// share of the pass (SOAR Nano at 1024^2, units of 2^14 to 2^19 elements,
// 1 x 1 convolution epilogues of 256 to 4096 partials: 4.204 ms per
// training step folding up to 128, 4.155 up to 2048).
constexpr int64_t kFoldAlways = 128;
constexpr int64_t kFoldBigUnit = (int64_t)1 << 20;

bool fold_fits(const Plan& p, const Tuning& t, int64_t partials) {
    return t.fold_max > 0 && partials <= std::min<int64_t>(t.fold_max, kFoldMax) &&
           (partials <= kFoldAlways || p.cpg * p.HW <= kFoldBigUnit);
}

bool fold_ok(const Plan& p, const Tuning& t, int64_t upb) {
    return fold_fits(p, t, p.cpg * p.cpp) && upb >= p.units;
}

// First chunk block of units [u0, u0 + nu) that loads with cached loads:
// the tail of about p.nt_tail bytes (over `tensors` tensors) that the
// reverse-walking second pass reads first, so it is still in the MALL.
// Blocks before it use non-temporal loads when p.ntl1 is set.
int64_t nt_end(const Plan& p, int64_t u0, int64_t nu, int tensors) {
    const int64_t bpu = p.cpg * p.cpp;
    const int64_t per_block = p.chunk * 4 * tensors;
    const int64_t tail = std::min(nu * bpu, (p.nt_tail + per_block - 1) / per_block);
    return (u0 + nu) * bpu - tail;
}

// First-pass kernels: `fin_nu` finish blocks for units [fin_u0, fin_u0 +
// fin_nu), then chunk blocks for units [u0, u0 + nu).
void launch_stats(const Plan& p, const FwdArgs& a, const WsView& w, int64_t fin_u0,
                  int64_t fin_nu, int64_t u0, int64_t nu, hipStream_t s) {
    const int64_t bpu = p.cpg * p.cpp;
    const dim3 grid((unsigned)(fin_nu + nu * bpu));
    const int tok = prof_begin(s, nu ? "gn_stats_partial" : "gn_stats_finish");
    if (nu == 0 && bpu >= kWideFinish) {
        k_stats_finish_wide<<<grid, kWideThreads, 0, s>>>(w.part, a.mean, a.rstd, a.mean_lo, w.lo,
                                                          p.HW, p.chunk, p.cpp, p.cpg, fin_u0,
                                                          a.eps);
        prof_end(s, tok);
        return;
    }
    bsel(p.vec4, [&](auto V) {
        loads_sel(p.loads, [&](auto U) {
            bsel(V() && p.ntl1, [&](auto L) {
                k_stats<V(), U(), L()><<<grid, kThreads, 0, s>>>(
                    a.x, w.part, a.mean, a.rstd, a.mean_lo, w.lo, p.HW, p.chunk, p.cpp, p.cpg,
                    fin_u0, fin_nu, u0 * bpu, a.eps, nt_end(p, u0, nu, 1));
            });
        });
    });
    prof_end(s, tok);
}

// The backward recovers the mean residual itself (finish_bwd_unit) when
// the caller saved none and there is no SiLU.
bool recover_lo(const BwdArgs& a) { return !a.mean_lo && !(a.flags & SOAR_GN_SILU); }

void launch_reduce(const Plan& p, const BwdArgs& a, const WsView& w, int64_t fin_u0,
                   int64_t fin_nu, int64_t u0, int64_t nu, hipStream_t s) {
    const int64_t bpu = p.cpg * p.cpp;
    const bool silu = (a.flags & SOAR_GN_SILU) != 0;
    const dim3 grid((unsigned)(fin_nu + nu * bpu));
    const int tok = prof_begin(s, nu ? (silu ? "gn_silu_bwd_reduce" : "gn_bwd_reduce")
                                     : "gn_bwd_finish");
    auto go = [&](auto V, auto S, auto L) {
        loads_sel(p.loads, [&](auto U) {
            bsel(V() && p.ntl1, [&](auto NL) {
                k_bwd_reduce<V(), S(), L(), U(), NL()><<<grid, kThreads, 0, s>>>(
                    a.dy, a.x, a.gamma, a.beta, a.mean, a.rstd, a.mean_lo, w.part, w.part_x,
                    w.lo, w.plane_sums, w.unit_sums, p.C, p.G, p.cpg, p.HW, p.chunk, p.cpp,
                    fin_u0, fin_nu, u0 * bpu, nt_end(p, u0, nu, 2));
            });
        });
    };
    bsel(p.vec4, [&](auto V) {
        if (silu)
            go(V, std::true_type{}, std::false_type{});
        else
            bsel(recover_lo(a), [&](auto L) { go(V, std::false_type{}, L); });
    });
    prof_end(s, tok);
}

// ---- two-stream pipeline --------------------------------------------------
// A helper stream (default priority) runs the first pass of batch b+1
// while the caller's stream runs the finish and second pass of batch b:
//
//   helper:  S0 --ev-- S1 --ev-- S2 ...            (S(b) waits for A(b-2))
//   caller:       F0 A0     F1 A1     F2 A2 ...
//
// Events fork the helper off the caller's stream and every helper kernel
// is waited on by the caller's stream, so when the call returns all work
// is ordered before anything later on the caller's stream.
struct Pipe {
    std::mutex mu;
    hipStream_t helper = nullptr;
    hipEvent_t fork = nullptr;
    hipEvent_t first[2] = {nullptr, nullptr};
    hipEvent_t second[4] = {nullptr, nullptr, nullptr, nullptr};
};

hipError_t pipe_for_device(Pipe** out) {
    static std::mutex mu;
    static Pipe* pipes[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!pipes[dev]) {
        Pipe* p = new Pipe;
        e = hipStreamCreateWithFlags(&p->helper, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&p->fork, hipEventDisableTiming);
        for (auto& ev : p->first)
            if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        for (auto& ev : p->second)
            if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return e;  // leaks the partial Pipe; the device is unusable anyway
        pipes[dev] = p;
    }
    *out = pipes[dev];
    return hipSuccess;
}

#define SOAR_TRY(x)                       \
    do {                                  \
        hipError_t e_ = (x);              \
        if (e_ != hipSuccess) return e_;  \
    } while (0)

int64_t units_per_batch(const Plan& p, const Tuning& t, int tensors_read) {
    if (t.batch_mb <= 0) return p.units;
    const double unit_bytes = (double)p.cpg * (double)p.HW * 4.0 * tensors_read;
    int64_t k = (int64_t)((double)t.batch_mb * 1048576.0 / unit_bytes);
    return std::max<int64_t>(1, std::min<int64_t>(k, p.units));
}

}  // namespace

bool make_plan(int64_t N, int64_t C, int64_t HW, int64_t G, const Tuning& t, Plan* p) {
    p->N = N;
    p->C = C;
    p->HW = HW;
    p->G = G;
    p->cpg = C / G;
    p->planes = N * C;
    p->units = N * G;
    // A chunk never exceeds the plane: small planes get one block each.
    const int64_t hw_up = (HW + 1023) / 1024 * 1024;
    p->chunk = t.chunk < hw_up ? t.chunk : hw_up;
    p->cpp = (HW + p->chunk - 1) / p->chunk;
    if (p->planes > (int64_t)0x7fffffff / p->cpp) return false;
    p->blocks = p->planes * p->cpp;
    p->chunk2 = t.chunk2 < hw_up ? t.chunk2 : hw_up;
    p->cpp2 = (HW + p->chunk2 - 1) / p->chunk2;
    if (p->planes > (int64_t)0x7fffffff / p->cpp2) return false;
    p->blocks2 = p->planes * p->cpp2;
    // a first-pass grid holds a batch's chunk blocks plus one finish block
    // per unit of the previous batch
    if (p->blocks + p->units > 0x7fffffff || C > 0x7fffffff) return false;
    p->vec4 = (HW % 4) == 0;
    p->loads = t.loads;
    p->ntl1 = (t.nt_load & 2) != 0;
    p->nt_tail = t.nt_tail_mb << 20;
    p->upb_fwd = units_per_batch(*p, t, 1);
    p->upb_bwd = units_per_batch(*p, t, 2);
    return true;
}

// Workspace regions, each 256-byte aligned:
//   chunk partials   double2 x blocks
//   plane sums       double2 x planes
//   unit S1/S2       double2 x units
//   mean residuals   float   x units
//   chunk sums of x - mu   double x blocks (backward without SiLU and
//                          without a saved mean residual)
size_t workspace_bytes(const Plan& p) {
    return align256(sizeof(double2) * (size_t)p.blocks) +
           align256(sizeof(double2) * (size_t)p.planes) +
           align256(sizeof(double2) * (size_t)p.units) +
           align256(sizeof(float) * (size_t)p.units) +
           align256(sizeof(double) * (size_t)p.blocks);
}

// Single-stream launch order for batches 0..B-1 (S = first pass, F =
// finish, A = second pass):  S0, F0+S1, A0, F1+S2, A1, ..., F(B-1), A(B-1).
// With two streams (tuning `streams` = 2 and more than one batch) the
// helper-stream pipeline above is used instead.
// The one-launch paths above apply when a unit is at most t.small_unit
// elements; the backward also bounds the samples a block walks.
// log2 of the threads per channel of the small kernels, or -1 when the
// unit does not fit: cpg rounded up to a power of two times HW must fit
// kSmallPer elements per thread.
int small_lg(const Plan& p, const Tuning& t, int nt) {
    if (t.small_unit <= 0 || p.cpg > kMaxSmallCpg || p.cpg * p.HW > t.small_unit) return -1;
    int lc = 0;
    while ((int64_t(1) << lc) < p.cpg) ++lc;
    int ln = 0;
    while ((1 << ln) < nt) ++ln;
    const int lg = ln - lc;  // log2(nt / cpgp)
    if (lg < 2 || p.HW > (int64_t)kSmallPer << lg) return -1;
    return lg;
}

// Threads of the small kernels' block for this plan: 256 when that many
// hold the unit, else 1024; 0 when the unit is not small.
int small_threads(const Plan& p, const Tuning& t) {
    if (small_lg(p, t, 256) >= 0) return 256;
    return small_lg(p, t, kSmallThreads) >= 0 ? kSmallThreads : 0;
}

// Runs f(std::integral_constant<int, NT>) for the plan's block size.
template <typename F>
void nt_sel(int nt, F&& f) {
    if (nt == 256)
        f(std::integral_constant<int, 256>{});
    else
        f(std::integral_constant<int, kSmallThreads>{});
}

bool small_fwd(const Plan& p, const Tuning& t) {
    return small_threads(p, t) > 0 && p.units <= 0x7fffffff;
}

bool small_bwd(const Plan& p, const Tuning& t) {
    return small_fwd(p, t) && p.N * p.cpg * p.HW <= 8 * t.small_unit && p.G <= 0x7fffffff;
}

hipError_t launch_forward(const Plan& p, const Tuning& t, const FwdArgs& a, hipStream_t s) {
    const WsView w = ws_view(p, a.ws);
    const bool silu = (a.flags & SOAR_GN_SILU) != 0;
    if (small_fwd(p, t)) {
        const int tok = prof_begin(s, "gn_small_fwd");
        const int nt = small_threads(p, t);
        nt_sel(nt, [&](auto NT) {
            bsel(silu, [&](auto S) {
                bsel((a.flags & SOAR_GN_RESIDUAL) != 0, [&](auto R) {
                    k_small_fwd<NT(), S(), R()><<<dim3((unsigned)p.units), NT(), 0, s>>>(
                        a.x, a.gamma, a.beta, a.y, a.mean, a.rstd, a.mean_lo, p.G, p.cpg, p.HW,
                        small_lg(p, t, nt), a.eps);
                });
            });
        });
        prof_end(s, tok);
        return hipGetLastError();
    }
    const int64_t bpu2 = p.cpg * p.cpp2;  // second-pass blocks per unit
    const char* apply_name = silu ? "gn_silu_apply" : "gn_apply";
    if (fold_ok(p, t, p.upb_fwd)) {
        launch_stats(p, a, w, 0, 0, 0, p.units, s);
        const int tok = prof_begin(s, apply_name);
        launch_apply(p, t, a, w.lo, 0, p.blocks2, s, kFoldChunks);
        prof_end(s, tok);
        return hipGetLastError();
    }
    if (t.streams >= 2 && p.units > p.upb_fwd) {
        Pipe* pp = nullptr;
        SOAR_TRY(pipe_for_device(&pp));
        std::lock_guard<std::mutex> lk(pp->mu);
        SOAR_TRY(hipEventRecord(pp->fork, s));
        SOAR_TRY(hipStreamWaitEvent(pp->helper, pp->fork, 0));
        int64_t bi = 0;
        for (int64_t u0 = 0; u0 < p.units; u0 += p.upb_fwd, ++bi) {
            const int64_t nu = std::min(p.upb_fwd, p.units - u0);
            if (bi >= 2) SOAR_TRY(hipStreamWaitEvent(pp->helper, pp->second[(bi - 2) % 4], 0));
            launch_stats(p, a, w, 0, 0, u0, nu, pp->helper);
            SOAR_TRY(hipEventRecord(pp->first[bi % 2], pp->helper));
            SOAR_TRY(hipStreamWaitEvent(s, pp->first[bi % 2], 0));
            launch_stats(p, a, w, u0, nu, 0, 0, s);
            const int tok = prof_begin(s, apply_name);
            launch_apply(p, t, a, w.lo, u0 * bpu2, nu * bpu2, s);
            prof_end(s, tok);
            SOAR_TRY(hipEventRecord(pp->second[bi % 4], s));
        }
        return hipGetLastError();
    }
    int64_t prev_u0 = 0, prev_nu = 0;
    for (int64_t u0 = 0;; u0 += p.upb_fwd) {
        const int64_t nu = u0 < p.units ? std::min(p.upb_fwd, p.units - u0) : 0;
        if (nu + prev_nu > 0) launch_stats(p, a, w, prev_u0, prev_nu, u0, nu, s);
        if (prev_nu > 0) {
            const int tok = prof_begin(s, apply_name);
            launch_apply(p, t, a, w.lo, prev_u0 * bpu2, prev_nu * bpu2, s);
            prof_end(s, tok);
        }
        if (nu == 0) break;
        prev_u0 = u0;
        prev_nu = nu;
    }
    return hipGetLastError();
}

hipError_t launch_forward_from_partials(const Plan& p, const Tuning& t, const FwdArgs& a,
                                        hipStream_t s) {
    const WsView w = ws_view(p, a.ws);
    if (small_fwd(p, t)) {
        const int tok = prof_begin(s, "gn_small_finish_apply");
        const int nt = small_threads(p, t);
        nt_sel(nt, [&](auto NT) {
            bsel((a.flags & SOAR_GN_SILU) != 0, [&](auto S) {
                bsel((a.flags & SOAR_GN_RESIDUAL) != 0, [&](auto R) {
                    k_small_finish_apply<NT(), S(), R()><<<dim3((unsigned)p.units), NT(), 0, s>>>(
                        a.x, a.gamma, a.beta, a.y, w.part, a.mean, a.rstd, a.mean_lo, w.lo, p.G,
                        p.cpg, p.HW, p.chunk, p.cpp, small_lg(p, t, nt), a.eps);
                });
            });
        });
        prof_end(s, tok);
        return hipGetLastError();
    }
    const bool fold = fold_fits(p, t, p.cpg * p.cpp);
    if (!fold) launch_stats(p, a, w, 0, p.units, 0, 0, s);
    const int tok = prof_begin(s, (a.flags & SOAR_GN_SILU) ? "gn_silu_apply" : "gn_apply");
    launch_apply(p, t, a, w.lo, 0, p.blocks2, s, fold ? kFoldChunks : 0);
    prof_end(s, tok);
    return hipGetLastError();
}

double2* ws_partials(const Plan& p, void* ws) { return ws_view(p, ws).part; }

bool forward_is_small(const Plan& p, const Tuning& t) { return small_fwd(p, t); }

hipError_t launch_forward_from_tile_partials(const Plan& p, const Tuning& t, const FwdArgs& a,
                                             const double2* part, const DwStatsGeom& g,
                                             int64_t Ho, int64_t Wo, hipStream_t s) {
    const WsView w = ws_view(p, a.ws);
    const int64_t P = p.cpg * g.tpp;
    const TileCount count{g.tpp, g.tiles_x, g.rows, Ho, Wo};
    if (fold_fits(p, t, P)) {
        const int tok = prof_begin(s, (a.flags & SOAR_GN_SILU) ? "gn_silu_apply" : "gn_apply");
        launch_apply(p, t, a, w.lo, 0, p.blocks2, s, kFoldTiles, part, count);
        prof_end(s, tok);
        return hipGetLastError();
    }
    int tok = prof_begin(s, "gn_stats_finish");
    if (P >= kWideFinish)
        k_stats_finish_tiles<kWideThreads><<<dim3((unsigned)p.units), kWideThreads, 0, s>>>(
            part, a.mean, a.rstd, a.mean_lo, w.lo, P, count, (double)(p.cpg * p.HW), a.eps);
    else
        k_stats_finish_tiles<kThreads><<<dim3((unsigned)p.units), kThreads, 0, s>>>(
            part, a.mean, a.rstd, a.mean_lo, w.lo, P, count, (double)(p.cpg * p.HW), a.eps);
    prof_end(s, tok);
    tok = prof_begin(s, (a.flags & SOAR_GN_SILU) ? "gn_silu_apply" : "gn_apply");
    launch_apply(p, t, a, w.lo, 0, p.blocks2, s);
    prof_end(s, tok);
    return hipGetLastError();
}

bool make_pw_plan(int64_t N, int64_t C_out, int64_t HW, int64_t G, const Tuning& t, Plan* p) {
    Tuning tp = t;
    tp.chunk = pw_pick_chunk(N, C_out, HW, t.pw_chunk);
    tp.batch_mb = 0;
    if (!make_plan(N, C_out, HW, G, tp, p)) return false;
    return p->chunk % 128 == 0;
}

// Same orders as the forward with R = reduction, D = dx, then the
// dgamma/dbeta finish over all planes.
bool backward_is_small(const Plan& p, const Tuning& t) { return small_bwd(p, t); }

bool backward_sums_foldable(const Plan& p, const Tuning& t, const BwdArgs& a, int64_t planes) {
    return !recover_lo(a) && planes <= kFoldPlanes && fold_fits(p, t, planes * p.cpp);
}

hipError_t launch_backward_sums(const Plan& p, const BwdArgs& a, hipStream_t s, BwdSums* out,
                                bool fold) {
    const WsView w = ws_view(p, a.ws);
    launch_reduce(p, a, w, 0, 0, 0, p.units, s);
    if (!fold) launch_reduce(p, a, w, 0, p.units, 0, 0, s);
    out->plane_sums = fold ? nullptr : w.plane_sums;
    out->unit_sums = fold ? nullptr : w.unit_sums;
    out->mean_lo = recover_lo(a) ? w.lo : a.mean_lo;
    out->part = w.part;
    out->cpp = p.cpp;
    return hipGetLastError();
}

hipError_t launch_backward(const Plan& p, const Tuning& t, const BwdArgs& a, hipStream_t s) {
    const WsView w = ws_view(p, a.ws);
    const bool silu = (a.flags & SOAR_GN_SILU) != 0;
    if (small_bwd(p, t)) {
        const int tok = prof_begin(s, "gn_small_bwd");
        const int nt = small_threads(p, t);
        const int lg = small_lg(p, t, nt);
        nt_sel(nt, [&](auto NT) {
            bsel(silu, [&](auto S) {
                bsel((a.flags & SOAR_GN_RESIDUAL) != 0, [&](auto R) {
                    bsel((a.flags & SOAR_GN_ACCUMULATE_DX) != 0, [&](auto A) {
                        bsel(p.HW <= ((int64_t)kSmallHalf << lg), [&](auto O) {
                            k_small_bwd<NT(), S(), R(), A(), O()>
                                <<<dim3((unsigned)p.G), NT(), 0, s>>>(
                                    a.dy, a.x, a.gamma, a.beta, a.mean, a.rstd, a.mean_lo, a.dx,
                                    a.dgamma, a.dbeta, p.N, p.C, p.G, p.cpg, p.HW, lg,
                                    recover_lo(a) ? 1 : 0);
                        });
                    });
                });
            });
        });
        prof_end(s, tok);
        return hipGetLastError();
    }
    const int64_t bpu2 = p.cpg * p.cpp2;  // second-pass blocks per unit
    const char* dx_name = silu ? "gn_silu_bwd_dx" : "gn_bwd_dx";
    const bool lorec = recover_lo(a);
    const bool params = a.dgamma || a.dbeta;
    // with the mean residual recovered, the dx pass reads it from the
    // workspace, where the finish put it
    BwdArgs ad = a;
    if (lorec) ad.mean_lo = w.lo;
    if (a.dx && !lorec && fold_ok(p, t, p.upb_bwd)) {
        launch_reduce(p, a, w, 0, 0, 0, p.units, s);
        const int tok = prof_begin(s, dx_name);
        launch_dx(p, t, a, w.unit_sums, 0, p.blocks2, s, true);
        prof_end(s, tok);
        return hipGetLastError();
    }
    bool param_in_dx = false;
    if (t.streams >= 2 && p.units > p.upb_bwd) {
        Pipe* pp = nullptr;
        SOAR_TRY(pipe_for_device(&pp));
        std::lock_guard<std::mutex> lk(pp->mu);
        SOAR_TRY(hipEventRecord(pp->fork, s));
        SOAR_TRY(hipStreamWaitEvent(pp->helper, pp->fork, 0));
        int64_t bi = 0;
        for (int64_t u0 = 0; u0 < p.units; u0 += p.upb_bwd, ++bi) {
            const int64_t nu = std::min(p.upb_bwd, p.units - u0);
            if (bi >= 2) SOAR_TRY(hipStreamWaitEvent(pp->helper, pp->second[(bi - 2) % 4], 0));
            launch_reduce(p, a, w, 0, 0, u0, nu, pp->helper);
            SOAR_TRY(hipEventRecord(pp->first[bi % 2], pp->helper));
            SOAR_TRY(hipStreamWaitEvent(s, pp->first[bi % 2], 0));
            launch_reduce(p, a, w, u0, nu, 0, 0, s);
            if (a.dx) {
                const int tok = prof_begin(s, dx_name);
                launch_dx(p, t, ad, w.unit_sums, u0 * bpu2, nu * bpu2, s);
                prof_end(s, tok);
            }
            SOAR_TRY(hipEventRecord(pp->second[bi % 4], s));
        }
    } else {
        // one batch: its dx launch runs after every plane sum is final, so
        // it also finishes dgamma / dbeta (no k_param_finish launch)
        param_in_dx = a.dx && params && p.units <= p.upb_bwd;
        int64_t prev_u0 = 0, prev_nu = 0;
        for (int64_t u0 = 0;; u0 += p.upb_bwd) {
            const int64_t nu = u0 < p.units ? std::min(p.upb_bwd, p.units - u0) : 0;
            if (nu + prev_nu > 0) launch_reduce(p, a, w, prev_u0, prev_nu, u0, nu, s);
            if (prev_nu > 0 && a.dx) {
                const int tok = prof_begin(s, dx_name);
                launch_dx(p, t, ad, w.unit_sums, prev_u0 * bpu2, prev_nu * bpu2, s, false,
                          param_in_dx ? w.plane_sums : nullptr);
                prof_end(s, tok);
            }
            if (nu == 0) break;
            prev_u0 = u0;
            prev_nu = nu;
        }
    }
    if (params && !param_in_dx) {
        const int tok = prof_begin(s, "gn_param_finish");
        k_param_finish<<<dim3((unsigned)((p.C + 255) / 256)), 256, 0, s>>>(
            w.plane_sums, a.dgamma, a.dbeta, p.N, p.C);
        prof_end(s, tok);
    }
    return hipGetLastError();
}

}  // namespace gn
}  // namespace soar
