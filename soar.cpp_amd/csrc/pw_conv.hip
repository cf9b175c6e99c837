// pw_conv.hip - pointwise (1x1, stride 1, no padding) convolution on the
// fp32 matrix cores of gfx950, with the GroupNorm statistics of its output
// computed in the epilogue.
//
// The convolution of one sample is a GEMM  z[co][p] = b[co] + sum_ci
// w[co][ci] * x[ci][p]  with the pixel axis p contiguous in HBM.  It runs on
// v_mfma_f32_32x32x2f32 (full fp32 products and sums, no reduced-precision
// inputs), so results stay within fp32 rounding of the reference's scalar
// loop (src/cuda/ops/convolution_kernels.cu:10-31, src/nn/layers.cpp
// :380-395).
//
// Work split.  One wave (a 64-thread block) owns one pixel chunk of one
// sample, cut into 128-pixel items, and computes every output row for it,
// 64 rows (two 32-row MFMA tiles) at a time.  Operand layout of the MFMA
// (lane l = 32*h + j):
//   a = W[row j of the tile][k = h]      b = X[k = h][pixel column j]
//   c[r] = Z[row (r%4) + 8*(r/4) + 4*h][pixel column j]
// The K axis is walked eight channels at a time: at k-step q half-wave h
// supplies channel 4h + q, so the four k-steps of one half read four
// consecutive channels of W with one 16-byte load.  Pixel column j of n-tile t is pixel
// 4*j + t of the item, so one 16-byte load of x gives lane j its b operand
// for all four n-tiles, and the four n-tile results of one row are again
// four consecutive pixels: z is written with 16-byte stores.
//
// GroupNorm statistics (optional).  For each row the epilogue shifts the
// item's values by the row's value at the item's first pixel (an exact
// data value, so differences stay small when |mean| >> std), sums the
// shifted values and their squares per lane, and transposes the per-lane
// sums through LDS so lane l ends up owning row l of the tile.  Lane l then
// folds the item into a float64 (count, mean, M2) triple with Chan's
// formula.  After the chunk, lane l writes the row's triple as the chunk
// partial part[(n*C_out + row)*cpp + chunk] - the layout the GroupNorm
// finish kernel combines - so GroupNorm needs no separate statistics pass
// over z.
#include <algorithm>
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
typedef float f16 __attribute__((ext_vector_type(16)));

constexpr int kRowTile = 64;    // output rows per pass (two 32-row tiles)
constexpr int kItem = 128;      // pixels per item (four 32-column tiles)
constexpr int kRowGroup = 4;    // row tiles whose statistics a lane keeps
constexpr int kKzStepsPerWave = 2;  // least K steps per wave split over blocks (1: same time)
constexpr int kKzTiles = 256;   // grids of fewer (64-row x chunk) tiles split K over blocks
constexpr int kLdsStride = 34;  // float2 per LDS row: 32 lanes + 2 pad
// Word 3 of a raw buffer descriptor on gfx9-family parts (gfx950 included):
// 32-bit float data format, no swizzle, no stride.
constexpr int kRsrcWord3 = 0x00020000;

struct Mom {
    double n, mean, m2;
};

__device__ __forceinline__ Mom chan_merge(const Mom& a, const Mom& b) {
    if (b.n == 0.0) return a;
    if (a.n == 0.0) return b;
    Mom r;
    r.n = a.n + b.n;
    const double f = b.n / r.n;
    const double d = b.mean - a.mean;
    r.mean = a.mean + d * f;
    r.m2 = a.m2 + b.m2 + d * d * a.n * f;
    return r;
}

// Row of the 64-row tile held in accumulator register r of m-tile mt by a
// lane of half-wave h.
__device__ __forceinline__ int tile_row(int mt, int r, int h) {
    return mt * 32 + (r & 3) + 8 * (r >> 2) + 4 * h;
}

// Modes of the convolution kernels (k_pw_conv below).
enum PwMode { kPlain = 0, kStats = 1, kAccum = 2, kPlainT = 3, kAccumT = 4 };

// Accumulators of an item start at the bias of their rows (zero without
// bias, and on split-K waves other than wave 0).  (The bias loads stay
// inside the item instead of being hoisted out of the pixel loop, where 32
// bias values would stay live in registers.)
template <bool BIAS>
__device__ __forceinline__ void pw_acc_init(f16 (&acc)[2][4], const float* __restrict__ bias,
                                            int64_t row0, int64_t rlim, int h, int v) {
    const float* bias_i = bias;
    asm volatile("" : "+s"(bias_i));
    const float* bb = bias_i + row0 + 4 * h;  // bias of tile row 4h
    const bool full = rlim >= kRowTile - 1;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int c = tile_row(mt, r, 0);
            float bv = 0.0f;
            if (BIAS && v == 0) bv = (full || c + 4 * h <= rlim) ? bb[c] : 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[mt][t][r] = bv;
        }
    }
}

// One K step (8 channels) of an item: 32 MFMAs, the four k-steps q of the
// two m-tiles and four n-tiles.
__device__ __forceinline__ void pw_mfma_step(f16 (&acc)[2][4], const f4 (&a)[2], const f4 (&b)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc[mt][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mt][q], b[q][t], acc[mt][t], 0,
                                                                  0, 0);
        }
    }
}

// Item epilogue: z rows of the tile (ACC modes add the old z) and, with
// STATS, the item's per-row shifts in ldsK and shifted (sum, sum of
// squares) per lane in lds, for the row-owner merge.
template <bool FAST, int MODE>
__device__ __forceinline__ void pw_item_epilogue(const f16 (&acc)[2][4], float* __restrict__ zs,
                                                 int64_t p0, int64_t HW, int64_t rlim, int h,
                                                 int j, int v, bool lane_px, uint32_t zo,
                                                 float2* lds, float* ldsK) {
    constexpr bool STATS = MODE == kStats, ACC = MODE == kAccum || MODE == kAccumT;
    // ---- epilogue.  The row offsets below are computed here, not hoisted
    // out of the item loop where 32 of them would stay live in registers.
    int64_t hw_e = HW;
    asm volatile("" : "+s"(hw_e));
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int tr0 = tile_row(mt, r, 0);  // half 1 holds row tr0 + 4
            float* zr = reinterpret_cast<float*>(
                reinterpret_cast<char*>(zs + (int64_t)tr0 * hw_e) + zo);
            if (v == 0 && tr0 + 4 * h <= rlim) {
                if (FAST) {
                    if (lane_px) {
                        f4 v = {acc[mt][0][r], acc[mt][1][r], acc[mt][2][r], acc[mt][3][r]};
                        if (ACC) v += *reinterpret_cast<const f4*>(zr);
                        *reinterpret_cast<f4*>(zr) = v;
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        if (p0 + 4 * j + t < HW) zr[t] = ACC ? zr[t] + acc[mt][t][r] : acc[mt][t][r];
                }
            }
        }
    }
    if (STATS) {
        // shift of each row: its value at the item's first pixel, which
        // lane j = 0 of each half-wave holds; passed on through LDS
        if (j == 0 && v == 0) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
                for (int r = 0; r < 16; ++r) ldsK[tile_row(mt, r, h)] = acc[mt][0][r];
            }
        }
        __syncthreads();
        if (v != 0) return;
        // LDS addresses: one lane base plus constants, formed here so they
        // are not hoisted out of the item loop
        int lb = 4 * h;
        asm volatile("" : "+v"(lb));
        const float* kb = ldsK + lb;
        float2* sb = lds + lb * kLdsStride + j;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int c = tile_row(mt, r, 0);
                const float K = kb[c];
                float s = 0.f, q = 0.f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const bool ok = FAST ? lane_px : (p0 + 4 * j + t < HW);
                    const float d = ok ? acc[mt][t][r] - K : 0.0f;
                    s += d;
                    q = fmaf(d, d, q);
                }
                sb[c * kLdsStride] = make_float2(s, q);
            }
        }
    }
}

// Row-owner merge of an item's statistics: lane l adds the shifted sums of
// tile row l (its 32 lanes' pairs in lds) and folds the item into the row's
// running (count, mean, M2) in float64 with Chan's formula.
__device__ __forceinline__ void pw_stats_merge(const float2* lds, const float* ldsK, Mom& run,
                                               int lane, int nvalid) {
    float S = 0.f, Q = 0.f;
    const float4* src = reinterpret_cast<const float4*>(lds + lane * kLdsStride);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 u = src[i];
        S += u.x + u.z;
        Q += u.y + u.w;
    }
    const double cnt = (double)nvalid;
    Mom m;
    m.n = cnt;
    m.mean = (double)ldsK[lane] + (double)S / cnt;
    m.m2 = fmax((double)Q - (double)S * (double)S / cnt, 0.0);
    run = chan_merge(run, m);
}

// One 64-row x 128-pixel item: z rows [row0, row0 + 64) of pixels
// [p0, p0 + 128) of sample n, plus (STATS) the item's per-row shifted sums
// transposed through LDS and the per-row shifts in ldsK.
//
// Addressing: every pointer below is uniform across the wave (scalar
// registers) and each lane adds a 32-bit byte offset, so the loads and
// stores use the scalar-base + vector-offset form and no 64-bit per-lane
// addresses are held.  K is walked in steps of 8 channels: at k-step q of
// step kk, half-wave h supplies channel kk + 4h + q.
//
// FAST (HW % 4 == 0, C_in % 8 == 0, 16-byte aligned x, w, z): no divergent
// branch in the K loop.  A lane past the end of the plane loads the plane's
// last 16 bytes and weight rows past C_out load row C_out - 1.  The general
// path guards every scalar access and loads zeros instead.
// kPlainT / kAccumT: kPlain / kAccum with the weights given transposed,
// element (row m, channel k) at w[k * C_out + m] (dx = W^T dz straight from
// W, no transpose kernel; the A operand then takes four 4-byte loads per
// row and K step instead of one 16-byte load).
template <bool FAST, int MODE, bool BIAS, int KS, int PD>
__device__ __forceinline__ void pw_item(const float* __restrict__ xs, const float* __restrict__ ws,
                                        const float* __restrict__ bias, float* __restrict__ zs,
                                        int64_t row0, int64_t p0, int h, int j, int64_t C_in,
                                        int64_t C_out, int64_t HW, int Kpad, int kb, int ke,
                                        int v, float2* lds, float* ldsK, float* red) {
    // xs = x + n*C_in*HW + p0, ws = w + row0*C_in, zs = z + (n*C_out + row0)*HW + p0
    constexpr bool TW = MODE == kPlainT || MODE == kAccumT;
    const bool lane_px = p0 + 4 * j < HW;
    const uint32_t hw4 = (uint32_t)HW * 4u;  // bytes per channel plane
    // lane byte offsets: x at channel 4h, pixel 4j (clamped into the plane)
    const uint32_t xo = (uint32_t)h * 4u * hw4 +
                        4u * (uint32_t)(lane_px ? 4 * j : (FAST ? (int)(HW - 4 - p0) : 0));
    const int64_t rlim = C_out - 1 - row0;  // last valid tile row
    const bool w0ok = j <= rlim, w1ok = 32 + j <= rlim;
    // A-operand byte offsets: row-major W (channels 4h..4h+3 of the row in
    // one 16-byte load), or with TW the row's element of channel 4h
    const uint32_t r0 = (uint32_t)(w0ok ? j : (int)rlim), r1 = (uint32_t)(w1ok ? 32 + j : (int)rlim);
    const uint32_t wo0 = TW ? (4u * h * (uint32_t)C_out + r0) * 4u : (r0 * (uint32_t)C_in + 4u * h) * 4u;
    const uint32_t wo1 = TW ? (4u * h * (uint32_t)C_out + r1) * 4u : (r1 * (uint32_t)C_in + 4u * h) * 4u;
    const uint32_t wq = (uint32_t)C_out * 4u;  // TW: bytes from one channel to the next
    const uint32_t zo = (uint32_t)h * 4u * hw4 + 16u * (uint32_t)j;

    f16 acc[2][4];
    pw_acc_init<BIAS>(acc, bias, row0, rlim, h, v);

    auto load_step = [&](int kk, f4 (&a)[2], f4 (&b)[4]) {
        if (FAST) {
            // Raw buffer loads: the descriptor holds the step's wave-uniform
            // base, each lane adds its 32-bit offset and the channel offset
            // q*HW*4 is a scalar.  A step past the end (kk >= Kpad) gets an
            // empty descriptor, so its loads return zeros without touching
            // memory.  Clamped lanes and rows load valid but unrelated data:
            // an MFMA output column depends only on its own b column and an
            // output row only on its own a row, so those values only reach
            // outputs that are neither stored nor counted in the statistics.
            const bool live = kk < Kpad;
            const int kc = live ? kk : 0;
            const auto rw = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(TW ? ws + (int64_t)kc * C_out : ws + kc), (short)0,
                live ? 0x7fffffff : 0, kRsrcWord3);
            const auto rx = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(xs + (int64_t)kc * HW), (short)0, live ? 0x7fffffff : 0,
                kRsrcWord3);
            if (TW) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // (the channel step as the scalar offset: no extra VGPRs)
                    a[0][q] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rw, wo0, q * wq, 0));
                    a[1][q] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rw, wo1, q * wq, 0));
                }
            } else {
                a[0] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo0, 0, 0));
                a[1] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo1, 0, 0));
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
                b[q] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo, q * hw4, 0));
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t ci = kk + 4 * h + q;
                const bool cv = ci < C_in;
                a[0][q] = (cv && w0ok) ? (TW ? ws[ci * C_out + j] : ws[(int64_t)j * C_in + ci]) : 0.0f;
                a[1][q] = (cv && w1ok) ? (TW ? ws[ci * C_out + 32 + j]
                                             : ws[(int64_t)(32 + j) * C_in + ci])
                                       : 0.0f;
                const float* xr = xs + ci * HW + 4 * j;
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    b[q][t] = (cv && p0 + 4 * j + t < HW) ? xr[t] : 0.0f;
            }
        }
    };
    auto mfma_step = [&](const f4 (&a)[2], const f4 (&b)[4]) { pw_mfma_step(acc, a, b); };
    // Ping-pong operand buffers: the loads of the next step are issued
    // before the MFMAs of the current one, so their latency hides behind 32
    // MFMAs.  Loads are never under a branch (past the end they load zeros,
    // or on the general path reload the last step) and buffers are never
    // copied, so the wait before each MFMA group covers only the older
    // buffer.  sched_group_barrier keeps the order (the scheduler would
    // otherwise sink each load next to its use).
    // This wave's K steps are [kb, ke) (split-K: KS waves share the item).
    const int klast = FAST ? ke : ke - 8;
    auto sched = [] {
        if (FAST) {
            __builtin_amdgcn_sched_group_barrier(0x020, TW ? 12 : 6, 0);  // the vector loads
            __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);  // then 32 MFMAs
        }
    };
    int kk = kb;
    if (PD == 1) {
        f4 a0[2], b0[4], a1[2], b1[4];
        load_step(kb, a0, b0);
        for (; kk + 8 < ke; kk += 16) {
            load_step(kk + 8, a1, b1);
            mfma_step(a0, b0);
            sched();
            load_step(min(kk + 16, klast), a0, b0);
            mfma_step(a1, b1);
            sched();
        }
        if (kk < ke) mfma_step(a0, b0);  // odd number of steps
    } else {
        // PD steps in flight: PD + 1 operand buffers in a ring, unrolled so
        // every index is a constant (the tail runs the steps left over from
        // the last round, already loaded)
        f4 A[PD + 1][2], B[PD + 1][4];
#pragma unroll
        for (int i = 0; i < PD; ++i) load_step(min(kb + 8 * i, klast), A[i], B[i]);
        for (; kk + 8 * PD < ke; kk += 8 * (PD + 1)) {
#pragma unroll
            for (int i = 0; i <= PD; ++i) {
                load_step(min(kk + 8 * (i + PD), klast), A[(i + PD) % (PD + 1)],
                          B[(i + PD) % (PD + 1)]);
                mfma_step(A[i], B[i]);
                sched();
            }
        }
#pragma unroll
        for (int i = 0; i < PD; ++i)
            if (kk + 8 * i < ke) mfma_step(A[i], B[i]);
    }

    if (KS > 1) {
        // Wave 0 adds the other waves' accumulators in wave order, one
        // m-tile at a time through LDS ([wave - 1][register][lane]:
        // consecutive lanes, consecutive words).
        const int lane = 32 * h + j;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            __syncthreads();
            if (v > 0) {
                float* dst = red + (v - 1) * 4096 + lane;
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[(t * 16 + r) * 64] = acc[mt][t][r];
            }
            __syncthreads();
            if (v == 0) {
                for (int w = 1; w < KS; ++w) {
                    const float* src = red + (w - 1) * 4096 + lane;
#pragma unroll
                    for (int t = 0; t < 4; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[mt][t][r] += src[(t * 16 + r) * 64];
                }
            }
        }
    }

    pw_item_epilogue<FAST, MODE>(acc, zs, p0, HW, rlim, h, j, v, lane_px, zo, lds, ldsK);
}

// MODE kPlain: z = w x + b;  kStats: also the GroupNorm chunk partials;
// kAccum: z += w x.  BIAS: bias is non-null.  KS waves per block split the
// K steps of every item (kseg channels each, wave 0 adds the others'
// accumulators in order and runs the epilogue): used when the output has
// too few tiles to occupy the chip.  PD: K steps whose loads are in flight
// while a step's MFMAs run (PD > 1 runs one wave per SIMD, which leaves
// room for the extra operand buffers and the accumulators in AGPRs; KS > 1
// and the general path too: at two waves per SIMD those variants spilled
// 21-89 registers).  Byte
// offsets inside one sample's planes must fit in 32 bits (checked by the
// host with pw_offsets_fit).  Cross-block split-K: block z of a grid with
// gridDim.z > 1 takes the K steps [z kzseg, (z + 1) kzseg) (its KS waves
// split them again) and writes its products to the slice z + z * zslice;
// k_pw_kz_reduce adds the slices.
template <bool FAST, int MODE, bool BIAS, int KS, int PD>
__global__ __launch_bounds__(64 * KS, PD > 1 || KS > 1 || !FAST ? 1 : 2) void k_pw_conv(
    const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ z, double2* __restrict__ part,
    int64_t C_in, int64_t C_out, int64_t HW, int64_t chunk, int64_t cpp, int Kpad, int rpw,
    int kseg, int kzseg, int64_t zslice) {
    __shared__ __attribute__((aligned(16))) float2 lds[kRowTile * kLdsStride];
    __shared__ float ldsK[kRowTile];            // per-row shifts of the item
    __shared__ Mom ldsM[kRowGroup * kRowTile];  // row-owner running moments
    __shared__ float red[KS > 1 ? (KS - 1) * 4096 : 1];  // split-K accumulators

    constexpr bool STATS = MODE == kStats;
    // (KS == 1: compile-time wave 0 and the whole K range)
    const int lane = threadIdx.x & 63, v = KS > 1 ? (int)threadIdx.x >> 6 : 0;
    const int h = lane >> 5, j = lane & 31;
    const int kzb = (int)blockIdx.z * kzseg, kze = min(Kpad, kzb + kzseg);
    const int kb = KS > 1 ? kzb + v * kseg : kzb, ke = KS > 1 ? min(kze, kb + kseg) : kze;
    z += (int64_t)blockIdx.z * zslice;
    const int64_t n = (int64_t)blockIdx.x / cpp;
    const int64_t kc = (int64_t)blockIdx.x - n * cpp;
    const int64_t px0 = kc * chunk;
    const int64_t pend = min(px0 + chunk, HW);
    // this wave's row tiles: [blockIdx.y * rpw, +rpw) of the R tiles
    const int64_t R = min<int64_t>((C_out + kRowTile - 1) / kRowTile, ((int64_t)blockIdx.y + 1) * rpw);
    const float* xn = x + n * C_in * HW;
    float* zn = z + n * C_out * HW;

    for (int64_t rg = (int64_t)blockIdx.y * rpw; rg < R; rg += kRowGroup) {
        const int nrt = (int)min<int64_t>(kRowGroup, R - rg);
        if (STATS && v == 0) {
#pragma unroll
            for (int g = 0; g < kRowGroup; ++g) ldsM[g * kRowTile + lane] = Mom{0.0, 0.0, 0.0};
        }
        for (int64_t p0 = px0; p0 < pend; p0 += kItem) {
            const int nvalid = (int)min<int64_t>(kItem, HW - p0);
            for (int g = 0; g < nrt; ++g) {
                const int64_t row0 = (rg + g) * kRowTile;
                constexpr bool TW = MODE == kPlainT || MODE == kAccumT;
                pw_item<FAST, MODE, BIAS, KS, PD>(xn + p0, TW ? w + row0 : w + row0 * C_in, bias,
                                               zn + row0 * HW + p0, row0, p0, h, j, C_in, C_out,
                                               HW, Kpad, kb, ke, v, lds, ldsK, red);
                if (STATS) {
                    __syncthreads();
                }
                if (STATS && v == 0) pw_stats_merge(lds, ldsK, ldsM[g * kRowTile + lane], lane, nvalid);
                if (STATS) __syncthreads();
            }
        }
        if (STATS && v == 0) {
            for (int g = 0; g < nrt; ++g) {
                const int64_t row = (rg + g) * kRowTile + lane;
                const Mom m = ldsM[g * kRowTile + lane];
                if (row < C_out) part[(n * C_out + row) * cpp + kc] = make_double2(m.mean, m.m2);
            }
        }
    }
}

// Streamed form of k_pw_conv's fast path for grids of one-wave blocks
// (KS = 1): the wave's items (row group, pixel item, row tile; k_pw_conv's
// order) follow one another without draining the operand pipeline.  The
// loads run kSd K steps ahead of the MFMAs across item boundaries, so the
// next item's first steps are in flight while an item's epilogue stores z,
// and, since the memory counter retires in issue order, the waits of the
// next item's MFMAs cover those earlier loads and not the stores issued
// after them.  The ring holds kSd + 1 steps, so an item's K steps must be a
// multiple of kSd + 1 (pw_stream_fits); the slot of each step is then a
// compile-time constant.  The next item's operands come from the same load
// code with its base pointers and lane offsets selected by a wave-uniform
// condition; after the last item the descriptors are empty and the loads
// return zeros without touching memory.  Blocks take their pixel chunks in
// the XCD-aware order of xcd_block.
constexpr int kSd = 3;

struct PwOff {
    uint32_t xo, wo0, wo1;  // lane byte offsets of x and of the two W rows
};

template <int MODE, bool BIAS>
__global__ __launch_bounds__(64, 1) void k_pw_conv_stream(
    const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ z, double2* __restrict__ part, int64_t C_in, int64_t C_out, int64_t HW,
    int64_t chunk, int64_t cpp, int Kpad, int rpw) {
    __shared__ __attribute__((aligned(16))) float2 lds[kRowTile * kLdsStride];
    __shared__ float ldsK[kRowTile];
    __shared__ Mom ldsM[kRowGroup * kRowTile];
    constexpr bool STATS = MODE == kStats, TW = MODE == kPlainT || MODE == kAccumT;
    constexpr int NB = kSd + 1;
    const int lane = threadIdx.x, h = lane >> 5, j = lane & 31;
    const int64_t bx = xcd_block(blockIdx.x, gridDim.x);  // the pixel chunk
    const int64_t n = bx / cpp;
    const int64_t kc = bx - n * cpp;
    const int64_t px0 = kc * chunk, pend = min(px0 + chunk, HW);
    const int64_t R = min<int64_t>((C_out + kRowTile - 1) / kRowTile, ((int64_t)blockIdx.y + 1) * rpw);
    const int64_t rg0 = (int64_t)blockIdx.y * rpw;
    if (rg0 >= R) return;
    const float* xn = x + n * C_in * HW;
    float* zn = z + n * C_out * HW;
    const uint32_t hw4 = (uint32_t)HW * 4u, wq = (uint32_t)C_out * 4u;
    const int nsteps = Kpad / 8;
    const uint32_t zo = (uint32_t)h * 4u * hw4 + 16u * (uint32_t)j;

    struct Task {
        int64_t rg, p0;
        int g;
    };
    auto next = [&](Task t) {
        if (++t.g >= (int)min<int64_t>(kRowGroup, R - t.rg)) {
            t.g = 0;
            t.p0 += kItem;
            if (t.p0 >= pend) {
                t.p0 = px0;
                t.rg += kRowGroup;
            }
        }
        return t;
    };
    auto row0_of = [](const Task& t) { return (t.rg + t.g) * kRowTile; };
    // k_pw_conv's lane offsets for a task (lanes past the plane and rows
    // past C_out are clamped onto valid addresses; their products reach no
    // stored output)
    auto offs = [&](const Task& t) {
        const int64_t rlim = C_out - 1 - row0_of(t);
        const bool lane_px = t.p0 + 4 * j < HW;
        const uint32_t r0 = (uint32_t)(j <= rlim ? j : (int)rlim);
        const uint32_t r1 = (uint32_t)(32 + j <= rlim ? 32 + j : (int)rlim);
        PwOff o;
        o.xo = (uint32_t)h * 4u * hw4 + 4u * (uint32_t)(lane_px ? 4 * j : (int)(HW - 4 - t.p0));
        o.wo0 = TW ? (4u * h * (uint32_t)C_out + r0) * 4u : (r0 * (uint32_t)C_in + 4u * h) * 4u;
        o.wo1 = TW ? (4u * h * (uint32_t)C_out + r1) * 4u : (r1 * (uint32_t)C_in + 4u * h) * 4u;
        return o;
    };
    auto load = [&](const float* xs, const float* ws, const PwOff& o, int kk, bool live,
                    f4 (&a)[2], f4 (&b)[4]) {
        const int k0 = live ? kk : 0;
        const auto rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(TW ? ws + (int64_t)k0 * C_out : ws + k0), (short)0,
            live ? 0x7fffffff : 0, kRsrcWord3);
        const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(xs + (int64_t)k0 * HW),
                                                          (short)0, live ? 0x7fffffff : 0,
                                                          kRsrcWord3);
        if (TW) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                a[0][q] = __builtin_bit_cast(float,
                                             __builtin_amdgcn_raw_buffer_load_b32(rw, o.wo0, q * wq, 0));
                a[1][q] = __builtin_bit_cast(float,
                                             __builtin_amdgcn_raw_buffer_load_b32(rw, o.wo1, q * wq, 0));
            }
        } else {
            a[0] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, o.wo0, 0, 0));
            a[1] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rw, o.wo1, 0, 0));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            b[q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, o.xo, q * hw4, 0));
    };
    auto wbase = [&](const Task& t) { return TW ? w + row0_of(t) : w + row0_of(t) * C_in; };

    if (STATS) {
#pragma unroll
        for (int g = 0; g < kRowGroup; ++g) ldsM[g * kRowTile + lane] = Mom{0.0, 0.0, 0.0};
    }
    Task cur{rg0, px0, 0};
    PwOff oc = offs(cur);
    const float* xc = xn + cur.p0;
    const float* wc = wbase(cur);
    f4 A[NB][2], B[NB][4];
#pragma unroll
    for (int i = 0; i < kSd; ++i) load(xc, wc, oc, 8 * i, true, A[i], B[i]);
    for (;;) {
        const Task nx = next(cur);
        const bool nv = nx.rg < R;
        const PwOff on = offs(nx);
        const float* xnx = xn + nx.p0;
        const float* wnx = wbase(nx);
        const int64_t row0 = row0_of(cur), rlim = C_out - 1 - row0;
        f16 acc[2][4];
        pw_acc_init<BIAS>(acc, bias, row0, rlim, h, 0);
        for (int s0 = 0; s0 < nsteps; s0 += NB) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int ls = s0 + i + kSd;  // the step loaded now
                const bool here = ls < nsteps;
                load(here ? xc : xnx, here ? wc : wnx, here ? oc : on, 8 * (here ? ls : ls - nsteps),
                     here || nv, A[(i + kSd) % NB], B[(i + kSd) % NB]);
                pw_mfma_step(acc, A[i], B[i]);
                __builtin_amdgcn_sched_group_barrier(0x020, TW ? 12 : 6, 0);  // the vector loads
                __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);           // then 32 MFMAs
            }
        }
        const bool lane_px = cur.p0 + 4 * j < HW;
        pw_item_epilogue<true, MODE>(acc, zn + row0 * HW + cur.p0, cur.p0, HW, rlim, h, j, 0,
                                     lane_px, zo, lds, ldsK);
        if (STATS) {
            __syncthreads();
            pw_stats_merge(lds, ldsK, ldsM[cur.g * kRowTile + lane], lane,
                           (int)min<int64_t>(kItem, HW - cur.p0));
            __syncthreads();
            if (!nv || nx.rg != cur.rg) {
                // the row group's chunk partials, then fresh moments
                const int nrt = (int)min<int64_t>(kRowGroup, R - cur.rg);
                for (int g = 0; g < nrt; ++g) {
                    const int64_t row = (cur.rg + g) * kRowTile + lane;
                    const Mom m = ldsM[g * kRowTile + lane];
                    if (row < C_out) part[(n * C_out + row) * cpp + kc] = make_double2(m.mean, m.m2);
                    ldsM[g * kRowTile + lane] = Mom{0.0, 0.0, 0.0};
                }
            }
        }
        if (!nv) break;
        cur = nx;
        oc = on;
        xc = xnx;
        wc = wnx;
    }
}

// Adds the KZ split-K slices of the convolution: z = bias + s_0 + s_1 + ...
// (+ the old z with ACC), slices in order.  One wave per (sample, output
// row, pixel chunk); with STATS it also writes the row's GroupNorm chunk
// partial part[(n*C_out + row)*cpp + chunk] = (mean, M2), shifted by the
// chunk's first value as the convolution epilogue does, the lanes' float
// sums combined in float64 by a fixed xor tree.
template <bool STATS, bool BIAS, bool ACC, bool V4>
__global__ __launch_bounds__(256) void k_pw_kz_reduce(const float* __restrict__ slices,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ z,
                                                      double2* __restrict__ part, int kz,
                                                      int64_t zslice, int64_t C_out, int64_t HW,
                                                      int64_t chunk, int64_t cpp) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= C_out) return;  // whole waves; no block barrier below
    const int64_t n = blockIdx.z, kc = blockIdx.x;
    const int64_t p0 = kc * chunk, p1 = min(p0 + chunk, HW);
    const int64_t base = (n * C_out + row) * HW;
    const float b = BIAS ? bias[row] : 0.0f;
    constexpr int V = V4 ? 4 : 1;
    float shift = 0.0f, s = 0.0f, q = 0.0f;
    for (int64_t p = p0 + (int64_t)lane * V; p < p1; p += 64 * V) {
        float v[V];
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = b;
        for (int k = 0; k < kz; ++k) {
            const float* src = slices + (int64_t)k * zslice + base + p;
            if (V4) {
                const float4 u = *reinterpret_cast<const float4*>(src);
                v[0] += u.x;
                v[1] += u.y;
                v[2] += u.z;
                v[3] += u.w;
            } else {
                v[0] += src[0];
            }
        }
        float* dst = z + base + p;
        if (ACC) {
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] += dst[e];
        }
        if (V4)
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        else
            dst[0] = v[0];
        if (STATS) {
            if (p == p0 + (int64_t)lane * V) shift = __shfl(v[0], 0);  // first round
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const float d = v[e] - shift;
                s += d;
                q = fmaf(d, d, q);
            }
        }
    }
    if (STATS) {
        double S = s, Q = q;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            S += __shfl_xor(S, off);
            Q += __shfl_xor(Q, off);
        }
        if (lane == 0) {
            const double cnt = (double)(p1 - p0);
            part[(n * C_out + row) * cpp + kc] =
                make_double2((double)shift + S / cnt, fmax(Q - S * S / cnt, 0.0));
        }
    }
}

// ======================================================================
// Weight and bias gradients: dW[co][ci] = sum_(n,p) dz[n][co][p] x[n][ci][p],
// db[co] = sum_(n,p) dz[n][co][p].  A GEMM whose K axis is the pixels:
// C[m = co][n = ci] = sum_k A[m][k] B[k][n], A = dz rows, B = x rows.
//
// One wave per (tile of dW: 64 x 64, or 32 rows / columns for a narrow
// matrix; pixel chunk of one sample).  Both MFMA operands put channels
// across lanes, so a step of 32 pixels is staged through LDS: the wave
// reads the tile's dz rows and x rows of the step with
// row-contiguous 16-byte loads (8 rows per instruction), writes them to LDS
// (row stride 144 bytes: conflict-free for the reads below), and each lane
// then reads its operand runs back (lane l = 32h + j: row j, pixels
// 16h + 4i .. +3 for k-steps (i, q)).  The next step's global loads are in
// flight during the current step's MFMAs.
// A block holds WPB waves on one pixel chunk of one sample, interleaved by
// step: wave w takes the steps at chunk start + 32 (w + WPB s), so the
// block's waves read adjacent 128-byte pieces of every row together (a
// 32 WPB-pixel run per row and block step).  Each wave has its own staging
// area and there is no barrier in the main loop.  At the end the waves
// park their accumulators in LDS and each adds a 1/WPB share of the tile
// over the WPB waves in wave order, so the block writes one fp32 partial
// tile (and, for the ci tile 0, the partial dz row sums) to the workspace:
// WPB times fewer partials than one per wave, which for deep layers are
// more bytes than the inputs.  A finish kernel adds the block partials in a
// fixed order in float64.
// ======================================================================
constexpr int kWgStep = 32;                 // pixels per step
constexpr int kWgStride = kWgStep + 4;      // floats per LDS row (144 bytes)

// TM, TN: 32-row MFMA tiles of dW along C_out and C_in (2 and 2: a 64 x 64
// tile; 1 when the matrix has at most 32 rows / columns, so a 16 x 32 dW
// does not pay for a 64 x 64 tile's MFMAs and loads).
template <bool FAST, int TM, int TN, int WPB>
__global__ __launch_bounds__(64 * WPB, 2) void k_pw_wgrad(
    const float* __restrict__ dz, const float* __restrict__ x, float* __restrict__ part_w,
    float* __restrict__ part_b, int64_t C_in, int64_t C_out, int64_t HW, int64_t chunk,
    int64_t cpp, int64_t tiles_ci) {
    constexpr int kStage = 2 * kRowTile * kWgStride;  // floats of one wave's staging
    constexpr int kR = 16 * TM * TN;                   // accumulators per lane
    static_assert(kR % WPB == 0 && WPB * kR * 64 <= WPB * kStage, "reduction layout");
    // per wave: rows 0..32TM-1: dz rows co0.., rows 64..64+32TN-1: x rows ci0..
    __shared__ __attribute__((aligned(16))) float lds_all[WPB * kStage];
    __shared__ float lds_b[WPB > 1 ? WPB * TM * 32 : 1];
    constexpr int kSlots = 4 * (TM + TN);  // load slots in use
    auto slot_used = [](int sl) { return sl < 8 ? sl < 4 * TM : sl - 8 < 4 * TN; };
    const int lane = threadIdx.x & 63;
    const int wv = WPB > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
    float* __restrict__ lds = lds_all + wv * kStage;
    const int h = lane >> 5, j = lane & 31;
    const int64_t tco = (int64_t)blockIdx.x / tiles_ci;
    const int64_t tci = (int64_t)blockIdx.x - tco * tiles_ci;
    const int64_t gb = blockIdx.y;  // n * cpp + chunk index (block partial)
    const int64_t n = gb / cpp, kc = gb - n * cpp;
    // this wave's first step; a wave with none loads nothing and adds zeros
    const int64_t px0 = kc * chunk + kWgStep * wv, pend = min(kc * chunk + chunk, HW);
    const int64_t co0 = tco * 32 * TM, ci0 = tci * 32 * TN;
    const bool want_b = tci == 0;

    // staging: load slot s (0..15) of lane l covers row 8s + l/8, pixels
    // 4*(l%8) .. +3 of the step (rows past the matrix are clamped to its last
    // row; their products reach only outputs that are not written)
    const int srow = lane >> 3, scol = 4 * (lane & 7);
    const float* src[16];
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) {
        const int r = 8 * sl + srow;  // 0..127
        if (r < kRowTile)
            src[sl] = dz + (n * C_out + min<int64_t>(co0 + r, C_out - 1)) * HW + scol;
        else
            src[sl] = x + (n * C_in + min<int64_t>(ci0 + r - kRowTile, C_in - 1)) * HW + scol;
    }
    auto gload = [&](int64_t p, f4 (&st)[16]) {
        const bool full = FAST && p + kWgStep <= pend;
#pragma unroll
        for (int sl = 0; sl < 16; ++sl) {
            if (!slot_used(sl)) continue;
            if (full) {
                st[sl] = *reinterpret_cast<const f4*>(src[sl] + p);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    st[sl][q] = p + scol + q < pend ? src[sl][p + q] : 0.0f;
            }
        }
    };
    auto lwrite = [&](const f4 (&st)[16]) {
#pragma unroll
        for (int sl = 0; sl < 16; ++sl)
            if (slot_used(sl))
                *reinterpret_cast<f4*>(&lds[(8 * sl + srow) * kWgStride + scol]) = st[sl];
    };

    f16 acc[TM][TN];
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.0f;
    float sb[TM];
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) sb[mt] = 0.0f;

    auto compute = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f4 A[TM], B[TN];
#pragma unroll
            for (int t = 0; t < TM; ++t)
                A[t] = *reinterpret_cast<const f4*>(
                    &lds[(32 * t + j) * kWgStride + 16 * h + 4 * i]);
#pragma unroll
            for (int t = 0; t < TN; ++t)
                B[t] = *reinterpret_cast<const f4*>(
                    &lds[(kRowTile + 32 * t + j) * kWgStride + 16 * h + 4 * i]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int mt = 0; mt < TM; ++mt)
#pragma unroll
                    for (int nt = 0; nt < TN; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(A[mt][q], B[nt][q],
                                                                           acc[mt][nt], 0, 0, 0);
            if (want_b) {
#pragma unroll
                for (int mt = 0; mt < TM; ++mt) sb[mt] += (A[mt][0] + A[mt][1]) + (A[mt][2] + A[mt][3]);
            }
        }
    };

    constexpr int64_t kStride = (int64_t)kWgStep * WPB;  // this wave's step stride
    f4 st[16];
    gload(px0, st);
    for (int64_t p = px0; p < pend; p += kStride) {
        lwrite(st);
        // next step's loads (the last step reloads itself: no branch, so the
        // wait before the LDS write above only covers these)
        const int64_t pn = p + kStride < pend ? p + kStride : p;
        gload(pn, st);
        if (FAST) {
            __builtin_amdgcn_sched_group_barrier(0x200, kSlots, 0);  // the LDS writes
            __builtin_amdgcn_sched_group_barrier(0x020, kSlots, 0);  // the global loads
        }
        compute();
    }

    if constexpr (WPB == 1) {
#pragma unroll
        for (int mt = 0; mt < TM; ++mt)
#pragma unroll
            for (int nt = 0; nt < TN; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t co = co0 + tile_row(mt, r, h);
                    const int64_t ci = ci0 + 32 * nt + j;
                    if (co < C_out && ci < C_in)
                        part_w[(gb * C_out + co) * C_in + ci] = acc[mt][nt][r];
                }
        if (want_b) {
#pragma unroll
            for (int mt = 0; mt < TM; ++mt) {
                const float tot = sb[mt] + __shfl_xor(sb[mt], 32);
                const int64_t co = co0 + 32 * mt + j;
                if (h == 0 && co < C_out) part_b[gb * C_out + co] = tot;
            }
        }
    } else {
        __syncthreads();  // every wave is done with its staging area
        // accumulator k = (mt * TN + nt) * 16 + r of wave w at red[(w kR + k) 64 + lane]
        float* __restrict__ red = lds_all;
#pragma unroll
        for (int mt = 0; mt < TM; ++mt)
#pragma unroll
            for (int nt = 0; nt < TN; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    red[(wv * kR + (mt * TN + nt) * 16 + r) * 64 + lane] = acc[mt][nt][r];
        if (want_b) {
#pragma unroll
            for (int mt = 0; mt < TM; ++mt) {
                const float tot = sb[mt] + __shfl_xor(sb[mt], 32);
                if (h == 0) lds_b[(wv * TM + mt) * 32 + j] = tot;
            }
        }
        __syncthreads();
        constexpr int kShare = kR / WPB;
#pragma unroll
        for (int kk = 0; kk < kShare; ++kk) {
            const int k = wv * kShare + kk;
            float t = red[k * 64 + lane];
#pragma unroll
            for (int w = 1; w < WPB; ++w) t += red[(w * kR + k) * 64 + lane];
            const int mt = k / (16 * TN), nt = (k / 16) % TN, r = k % 16;
            const int64_t co = co0 + tile_row(mt, r, h);
            const int64_t ci = ci0 + 32 * nt + j;
            if (co < C_out && ci < C_in) part_w[(gb * C_out + co) * C_in + ci] = t;
        }
        if (want_b && wv == 0 && h == 0) {
#pragma unroll
            for (int mt = 0; mt < TM; ++mt) {
                float t = lds_b[mt * 32 + j];
#pragma unroll
                for (int w = 1; w < WPB; ++w) t += lds_b[(w * TM + mt) * 32 + j];
                const int64_t co = co0 + 32 * mt + j;
                if (co < C_out) part_b[gb * C_out + co] = t;
            }
        }
    }
}

// ======================================================================
// Fused backward of a pointwise CBA block (1x1 convolution without bias,
// then GroupNorm, then optionally SiLU; blocks.cpp:429-445).  From the
// GroupNorm input z, the upstream gradient dy and the convolution input x
// one pass computes
//   dz = A_c dzs + D_u xhat + B_u   k_bwd_dx's arithmetic, dzs = dy or
//                                   dy silu'(gamma xhat + beta)
//   dx = W^T dz                     the convolution's input gradient
//   dW partial = sum dz x^T         one fp32 partial tile per block
// so dz is never written to HBM and read back: four tensor passes (z, dy
// and x in, dx out) instead of seven (GroupNorm dx 3, dgrad 2, wgrad 2).
// C_in, C_out <= 64 (one dW tile); the GroupNorm reduction and its finish
// run first and leave the per-unit S1 / S2 in unit_sums.
//
// Block = kFbPairs producer waves and kFbPairs consumer waves on one pixel
// chunk of one sample (two waves per SIMD).  The chunk is walked in windows
// of kFbPairs 32-pixel pieces, piece q being pair q's step.  The producers
// load a window together, two windows ahead, with row-contiguous 16-byte
// loads (k_pw_wgrad's slots: eight rows of 128 bytes per load) through
// buffer descriptors bounded to the sample's planes; a lane's eight rows
// are taken at piece (q + lane group) % kFbPairs, so one load touches four
// offsets of the planes instead of one (eight rows at one offset of planes
// a power of two apart meet one memory channel; a read of this shape took
// 682 us for 3 GiB with one offset per load, 450 us with four).  Each lane
// forms dz in registers from per-channel coefficients in LDS and writes its
// dz and x rows into the stage of the piece's pair (two stages per pair,
// k_pw_wgrad's layout).  One block barrier per window hands the stages to
// the consumers; consumer q then runs, for its piece,
//   dW: k_pw_wgrad's MFMAs, A = dz rows, B = x rows, K = the 32 pixels;
//   dx: C[ci][p] = sum_co W[co][ci] dz[co][p], A = W^T from registers
//       (lane (h, j) holds W[2s + h][32 t + j], zero for co >= C_out),
//       B = dz[2s + h][pixel j] read from LDS, K = the C_out channels, so
//       lane (h, j) ends with pixel j of rows tile_row(t, r, h), stored as
//       128-byte row pieces,
// while the producers form the next window.  (The producers' vector ALU
// work and the consumers' MFMAs do not run at the same time on a SIMD:
// fp32 MFMAs and VALU instructions of two waves of one SIMD take the sum of
// their times.  The split serves the shared, permuted loads.)  At the end
// the consumers add their dW tiles through LDS in pair order and the block
// writes one partial for k_sum_partials (at its chunk's index: blocks take
// their chunks in the XCD-aware order of xcd_block).  Block 0 also adds
// dgamma / dbeta from the plane sums, in k_param_finish's order.
// ======================================================================
constexpr int kFbPairs = 4;
// Cache policy of the buffer accesses: non-temporal (each byte is touched
// once; at 64 -> 64 channels over 2048^2 pixels 1065 -> 1033 us).
constexpr int kNt = 2;

template <bool SILU, int TM, int TN, bool ACC, bool FULL>
__global__ __launch_bounds__(128 * kFbPairs, 1) void k_pw_cba_bwd(
    const float* __restrict__ dy, const float* __restrict__ z, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ mean_lo,
    const double2* __restrict__ unit_sums, const double2* __restrict__ plane_sums,
    float* __restrict__ dgamma, float* __restrict__ dbeta, float* __restrict__ dx,
    float* __restrict__ part_w, int64_t C_in, int64_t C_out, int64_t HW, int64_t G,
    int64_t N, int64_t chunk, int64_t cpp, const double2* __restrict__ gn_part,
    int64_t gn_cpp) {
    constexpr int kZr = 32 * TM, kXr = 32 * TN;      // staged dz rows, x rows
    constexpr int kStage = (kZr + kXr) * kWgStride;  // floats of one stage
    constexpr int kR = 16 * TM * TN;                 // dW accumulators per lane
    static_assert(kR * 64 * kFbPairs <= 2 * kFbPairs * kStage, "reduction layout");
    __shared__ __attribute__((aligned(16))) float lds_all[2 * kFbPairs * kStage];
    __shared__ __attribute__((aligned(16))) float coef[64 * 8];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const bool producer = wv < kFbPairs;  // wave-uniform
    const int pr = producer ? wv : wv - kFbPairs;
    float* __restrict__ stages = lds_all + pr * 2 * kStage;
    const int h = lane >> 5, j = lane & 31;
    const int64_t bx = xcd_block(blockIdx.x, gridDim.x);  // the pixel chunk
    const int64_t n = bx / cpp, kc = bx - n * cpp;
    const int64_t cpg = C_out / G;

    // Without unit_sums the block folds the GroupNorm backward's finish:
    // the sums of sample n's planes (and, in block 0, of every sample's for
    // dgamma / dbeta) from the reduction's partials, into shared memory
    // the stages have not used yet, with the finish's own arithmetic.
    const bool fold = unit_sums == nullptr;  // block-uniform
    double2* fps = reinterpret_cast<double2*>(lds_all);  // [64] this sample's planes
    double2* fpq = fps + 64;                             // [64] sample s's, block 0
    float* fgam = reinterpret_cast<float*>(fps + 128);   // [64] their gamma
    if (fold) {
        bwd_plane_sums<128 * kFbPairs>(gn_part, (int)(n * C_out), (int)C_out, (int)gn_cpp, fps,
                                       gamma, (int)C_out, fgam);
        __syncthreads();
    }
    // Channel c's coefficients for sample n, as k_bwd_dx forms them:
    // mu, r, e, gamma, beta, A = gamma r, B = -r S1 / M, D = -r S2 / M
    // (zeros past C_out: those rows get dz = 0).
    if (threadIdx.x < 64) {
        const int c = threadIdx.x;
        f4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
        if (c < C_out) {
            const int64_t u = n * G + c / cpg;
            const float mu = mean[u], r = rstd[u];
            const float e = mean_lo ? -mean_lo[u] * r : 0.0f;
            const float gm = gamma ? gamma[c] : 1.0f, bt = beta ? beta[c] : 0.0f;
            const int64_t g0 = (u - n * G) * cpg;  // the unit's first plane in the sample
            const double2 S = fold ? bwd_unit_sums(fps + g0, fgam + g0, (int)cpg, (int)gn_cpp)
                                   : unit_sums[u];
            const double Md = (double)(cpg * HW);
            lo = f4{mu, r, e, gm};
            hi = f4{bt, gm * r, (float)(-(double)r * S.x / Md), (float)(-(double)r * S.y / Md)};
        }
        *reinterpret_cast<f4*>(&coef[8 * c]) = lo;
        *reinterpret_cast<f4*>(&coef[8 * c + 4]) = hi;
    }
    if (blockIdx.x == 0 && (dgamma || dbeta)) {
        // k_param_finish for channel c: the same sums in sample order
        const int64_t c = threadIdx.x;
        double sa = 0.0, sb = 0.0;
        for (int64_t s = 0; s < N; ++s) {
            double2 v;
            if (fold) {  // block-uniform
                bwd_plane_sums<128 * kFbPairs>(gn_part, (int)(s * C_out), (int)C_out,
                                               (int)gn_cpp, fpq);
                __syncthreads();
                if (c < C_out) v = fpq[c];
                __syncthreads();
            } else if (c < C_out) {
                v = plane_sums[s * C_out + c];
            }
            if (c < C_out) {
                sa += v.x;
                sb += v.y;
            }
        }
        if (c < C_out) {
            if (dbeta) dbeta[c] = (float)((double)dbeta[c] + sa);
            if (dgamma) dgamma[c] = (float)((double)dgamma[c] + sb);
        }
    }
    __syncthreads();

    const bool want_dx = dx != nullptr, want_dw = part_w != nullptr;  // block-uniform
    const uint32_t hw4 = (uint32_t)HW * 4u;
    const int64_t cbeg = kc * chunk, pend = min(cbeg + chunk, HW);
    constexpr int64_t kStride = (int64_t)kWgStep * kFbPairs;
    // block barriers: one per step of the longest pair, plus one to drain
    const int64_t iters = (pend - cbeg + kStride - 1) / kStride;

    f16 accw[TM][TN];
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) accw[mt][nt][r] = 0.0f;

    if (producer) {
        // staging slots (k_pw_wgrad's): slot sl of lane l covers row
        // 8 sl + l/8, pixels 4 (l % 8) .. +3 of the step
        const int srow = lane >> 3, scol = 4 * (lane & 7);
        const auto rz = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(z + n * C_out * HW),
                                                          (short)0, (int)(C_out * HW * 4), kRsrcWord3);
        const auto rg = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(dy + n * C_out * HW),
                                                          (short)0, (int)(C_out * HW * 4), kRsrcWord3);
        const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x + n * C_in * HW),
                                                          (short)0, (int)(C_in * HW * 4), kRsrcWord3);
        // two register sets: the loads run two steps ahead of the dz
        // work, so a step's loads have a whole step to arrive
        f4 az[4 * TM], ag[4 * TM], ax[4 * TN], bz[4 * TM], bg[4 * TM], bx[4 * TN];
        // The descriptor's range check covers the vector offset only: the
        // scalar offset is added to the address unchecked.  C_in and C_out
        // are multiples of 8 (pw_cba_fused_fits), so an 8-row slot lies
        // wholly inside or wholly past its tensor's rows; a slot past the
        // end takes the last 8 rows' scalar offset instead, so no load
        // leaves the sample.  Its values are harmless: a z/dy row past
        // C_out has zero coefficients, so its dz is 0 (for finite inputs; a
        // non-finite input makes its whole group NaN anyway), and an x row
        // past C_in only reaches dW columns that are never stored.
        // FULL (C_out = 32 TM and C_in = 32 TN, e.g. 64 -> 64): every slot
        // is a real row, so the offsets are the plain multiples of 8 rows.
        const uint32_t zlim = (uint32_t)C_out - 8u, xlim = (uint32_t)C_in - 8u;
        // The block's window of kFbPairs 32-pixel pieces (one per pair's
        // step) is loaded by all producers together: lane group g of
        // producer q takes its rows at piece (q + g) % kFbPairs, so the
        // eight rows of one 16-byte load lie at four different offsets of
        // their planes.  (Eight rows at one offset of planes a power of two
        // apart meet the same memory channel: one load's lines are then
        // served one after another.  A read of this shape took 682 us for
        // 3 GiB with one offset per load and 450 us with four.)  The lane
        // writes its rows into the stage of the pair that owns the piece.
        const int piece = (pr + srow) % kFbPairs;
        float* __restrict__ pstages = lds_all + piece * 2 * kStage;
        auto gload = [&](int64_t wb, f4 (&sz)[4 * TM], f4 (&sg)[4 * TM], f4 (&sx)[4 * TN]) {
            // lanes past the plane read its last 16 bytes (zeroed below)
            const uint32_t q = (uint32_t)min<int64_t>(wb + kWgStep * piece + scol, HW - 4);
            const uint32_t vo = (uint32_t)srow * hw4 + 4u * q;
            if constexpr (FULL) {
                const uint32_t row8 = 8u * hw4;
#pragma unroll
                for (int sl = 0; sl < 4 * TM; ++sl) {
                    sz[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rz, vo, sl * row8, kNt));
                    sg[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rg, vo, sl * row8, kNt));
                }
#pragma unroll
                for (int sl = 0; sl < 4 * TN; ++sl)
                    sx[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rx, vo, sl * row8, kNt));
            } else {
                // (the slots' scalar offsets are recomputed here on every
                // step, a few scalar instructions, rather than hoisted into
                // 16 registers)
                uint32_t h4 = hw4, zl = zlim, xl = xlim;
                asm volatile("" : "+s"(h4), "+s"(zl), "+s"(xl));
#pragma unroll
                for (int sl = 0; sl < 4 * TM; ++sl) {
                    const uint32_t so = min(8u * sl, zl) * h4;
                    sz[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rz, vo, so, kNt));
                    sg[sl] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rg, vo, so, kNt));
                }
#pragma unroll
                for (int sl = 0; sl < 4 * TN; ++sl)
                    sx[sl] = __builtin_bit_cast(
                        f4, __builtin_amdgcn_raw_buffer_load_b128(rx, vo, min(8u * sl, xl) * h4, kNt));
            }
        };
        // dz and x of the lane's piece of the window at wb into LDS stage st
        // of the piece's pair
        auto form = [&](int64_t wb, float* __restrict__ st, const f4 (&sz)[4 * TM],
                        const f4 (&sg)[4 * TM], const f4 (&sx)[4 * TN]) {
            // all four pixels or none (HW % 4 == 0)
            const bool live = wb + kWgStep * piece + scol < pend;
#pragma unroll
            for (int sl = 0; sl < 4 * TM; ++sl) {
                const int co = 8 * sl + srow;
                const f4 c0 = *reinterpret_cast<const f4*>(&coef[8 * co]);
                const f4 c1 = *reinterpret_cast<const f4*>(&coef[8 * co + 4]);
                f4 o;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float xh = fmaf(sz[sl][t] - c0[0], c0[1], c0[2]);
                    const float dzs = SILU ? dsilu_fast(sg[sl][t], fmaf(c0[3], xh, c1[0])) : sg[sl][t];
                    o[t] = live ? fmaf(c1[1], dzs, fmaf(c1[3], xh, c1[2])) : 0.0f;
                }
                *reinterpret_cast<f4*>(&st[(8 * sl + srow) * kWgStride + scol]) = o;
            }
#pragma unroll
            for (int sl = 0; sl < 4 * TN; ++sl) {
                const f4 v = live ? sx[sl] : f4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f4*>(&st[(kZr + 8 * sl + srow) * kWgStride + scol]) = v;
            }
        };
        // Windows alternate between the register sets (a and b) and the
        // LDS stages (0 and 1); a set is refilled with the window two ahead
        // right after its window is formed (a wave-uniform branch: windows
        // past the chunk load nothing).  iters + 1 barriers, as the
        // consumer.
        int64_t wb = cbeg;
        gload(wb, az, ag, ax);
        gload(wb + kStride, bz, bg, bx);
        for (int64_t i = 0; i <= iters; i += 2) {
            if (i < iters) {
                form(wb, pstages, az, ag, ax);
                if (wb + 2 * kStride < pend) gload(wb + 2 * kStride, az, ag, ax);
                wb += kStride;
            }
            lds_barrier();
            if (i + 1 <= iters) {
                if (i + 1 < iters) {
                    form(wb, pstages + kStage, bz, bg, bx);
                    if (wb + 2 * kStride < pend) gload(wb + 2 * kStride, bz, bg, bx);
                    wb += kStride;
                }
                lds_barrier();
            }
        }
    } else {
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(want_dx ? dx + n * C_in * HW : dx,
                                                          (short)0, (int)(C_in * HW * 4), kRsrcWord3);
        // W^T operand of dx: k-step s, half h -> channel co = 2s + h
        float wt[TN][16 * TM];
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int s = 0; s < 16 * TM; ++s) {
                const int64_t co = 2 * s + h, ci = 32 * t + j;
                wt[t][s] = (co < C_out && ci < C_in) ? w[co * C_in + ci] : 0.0f;
            }
        f16 accx[TN];
        int64_t p = cbeg + kWgStep * pr;
        for (int64_t i = 0; i <= iters; ++i) {
            if (i > 0) {
                // step i - 1 of the pair, at pixels p .. p + 31
                const float* __restrict__ st = stages + ((i - 1) & 1) * kStage;
                // dW += dz x^T over the step's 32 pixels
                if (want_dw) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        f4 A[TM], B[TN];
#pragma unroll
                        for (int t = 0; t < TM; ++t)
                            A[t] = *reinterpret_cast<const f4*>(&st[(32 * t + j) * kWgStride + 16 * h + 4 * k]);
#pragma unroll
                        for (int t = 0; t < TN; ++t)
                            B[t] = *reinterpret_cast<const f4*>(
                                &st[(kZr + 32 * t + j) * kWgStride + 16 * h + 4 * k]);
#pragma unroll
                        for (int q = 0; q < 4; ++q)
#pragma unroll
                            for (int mt = 0; mt < TM; ++mt)
#pragma unroll
                                for (int nt = 0; nt < TN; ++nt)
                                    accw[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                        A[mt][q], B[nt][q], accw[mt][nt], 0, 0, 0);
                    }
                }
                if (want_dx) {
                    // dx = W^T dz for the step's 32 pixels
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r) accx[t][r] = 0.0f;
#pragma unroll
                    for (int s = 0; s < 16 * TM; ++s) {
                        const float b = st[(2 * s + h) * kWgStride + j];
#pragma unroll
                        for (int t = 0; t < TN; ++t)
                            accx[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(wt[t][s], b, accx[t], 0, 0, 0);
                    }
                    if (p + j < pend) {
                        // Row 4h + c of the tile: with C_in a multiple of 8
                        // its test reduces to the wave-uniform
                        // 32 t + 8 (r / 4) < C_in, so the stores of rows
                        // past C_in are skipped by a scalar branch (the
                        // scalar row offset is not range-checked).
                        const uint32_t vo = (uint32_t)(4 * h) * hw4 + 4u * (uint32_t)(p + j);
#pragma unroll
                        for (int t = 0; t < TN; ++t)
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                if (!FULL && 32 * t + 8 * (r >> 2) >= C_in) continue;
                                const uint32_t so = (uint32_t)tile_row(t, r, 0) * hw4;
                                float v = accx[t][r];
                                if (ACC)
                                    v += __builtin_bit_cast(
                                        float, __builtin_amdgcn_raw_buffer_load_b32(ro, vo, so, 0));
                                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), ro, vo,
                                                                      so, kNt);
                            }
                    }
                }
                p += kStride;
            }
            lds_barrier();
        }
    }

    if (!want_dw) return;
    // the consumers' dW tiles added in pair order (k_pw_wgrad's reduction);
    // the last barrier above ended every read of the stages
    float* __restrict__ red = lds_all;
    if (!producer) {
#pragma unroll
        for (int mt = 0; mt < TM; ++mt)
#pragma unroll
            for (int nt = 0; nt < TN; ++nt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    red[(pr * kR + (mt * TN + nt) * 16 + r) * 64 + lane] = accw[mt][nt][r];
    }
    __syncthreads();
    if (producer) return;
    constexpr int kShare = kR / kFbPairs;
#pragma unroll
    for (int kk = 0; kk < kShare; ++kk) {
        const int k = pr * kShare + kk;
        float t = red[k * 64 + lane];
#pragma unroll
        for (int v = 1; v < kFbPairs; ++v) t += red[(v * kR + k) * 64 + lane];
        const int mt = k / (16 * TN), nt = (k / 16) % TN, r = k % 16;
        const int64_t co = tile_row(mt, r, h), ci = 32 * nt + j;
        if (co < C_out && ci < C_in) part_w[(bx * C_out + co) * C_in + ci] = t;
    }
}

// out[e] += sum_g part[g][e] for e < E, in float64 and a fixed order.  A
// block of 16 waves owns 64 consecutive columns: wave w adds rows
// [w*G/16, (w+1)*G/16) with each lane on one column (a 256-byte row segment
// per load, eight loads in flight), then the 16 wave sums are added in
// order.
// Two tables in one launch: blocks [0, nb0) add table 0 (part0 -> out0, E0
// entries), the rest table 1 (the dW and db partials of one weight
// gradient).
__global__ __launch_bounds__(1024) void k_sum_partials(const float* __restrict__ part0,
                                                       float* __restrict__ out0, int64_t E0,
                                                       int64_t nb0,
                                                       const float* __restrict__ part1,
                                                       float* __restrict__ out1, int64_t E1,
                                                       int64_t G) {
    __shared__ double lds[16][64];
    const bool first = (int64_t)blockIdx.x < nb0;
    const float* __restrict__ part = first ? part0 : part1;
    float* __restrict__ out = first ? out0 : out1;
    const int64_t E = first ? E0 : E1;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t e = ((int64_t)blockIdx.x - (first ? 0 : nb0)) * 64 + lane;
    const int64_t g0 = wv * G / 16, g1 = (wv + 1) * G / 16;
    const double sum = e < E ? segment_sum(part, E, e, g0, g1) : 0.0;
    lds[wv][lane] = sum;
    __syncthreads();
    if (wv == 0 && e < E) {
        double t = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) t += lds[i][lane];
        out[e] = (float)((double)out[e] + t);
    }
}

// wt[ci][co] = w[co][ci]
__global__ void k_transpose(const float* __restrict__ w, float* __restrict__ wt, int64_t R,
                            int64_t Cc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= R * Cc) return;
    const int64_t r = i / Cc, c = i - r * Cc;
    wt[c * R + r] = w[i];
}

// ======================================================================
// Small convolutions (Tuning::pw_small).  The MFMA kernels above give a
// wave a 64-row x 128-pixel tile and walk all of K on it; a small output
// has few such tiles, so a few waves run K/8 dependent MFMA steps each
// (about 0.1 us per channel of K) while the chip idles, and on planes of a
// few pixels most of each tile is empty.  Here one lane owns one output element z[n][m][p]
// (64 consecutive elements of a sample per wave: pixels fastest, then rows)
// and the K axis is split over the S waves of a block: wave v sums its
// contiguous k segment in fp32, then wave 0 adds the S partial sums in
// order and the bias (or adds the total to z with ACC).
//
// TRANS reads the weight as w[k][m], so dx = W^T dz needs no transposed
// copy.  V4 (not TRANS; K and the segment a multiple of 4, w 16-byte
// aligned) reads four weights of a row with one 16-byte load.  Element
// offsets inside one sample fit in 32 bits (checked by pw_small_fits).
// ======================================================================
constexpr int kSmallMaxWaves = 16;

// The body for output group `bx` (64 elements) of sample n; the block's
// blockDim.x / 64 waves split K.
template <bool TRANS, bool V4, bool ACC, bool BIAS>
__device__ __forceinline__ void pw_small_body(const float* __restrict__ x,
                                              const float* __restrict__ w,
                                              const float* __restrict__ bias,
                                              float* __restrict__ z, int M, int K, int HW,
                                              int seg, int64_t bx, int64_t n,
                                              float (*part)[64]) {
    const int lane = threadIdx.x & 63, v = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    const int MH = M * HW;
    const int o = (int)bx * 64 + lane;  // element of the sample's output
    const bool live = o < MH;
    const int oc = live ? o : MH - 1;  // lanes past the end compute a copy
    const int m = oc / HW, p = oc - m * HW;
    const float* xs = x + n * (int64_t)K * HW + p;
    const int k0 = v * seg, k1 = min(K, k0 + seg);
    float acc = 0.0f;
    int k = k0;
    if (V4) {
        const float* wr = w + (int64_t)m * K;
        for (; k + 8 <= k1; k += 8) {
            const float4 wa = *reinterpret_cast<const float4*>(wr + k);
            const float4 wb = *reinterpret_cast<const float4*>(wr + k + 4);
            float xv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) xv[u] = xs[(k + u) * HW];
            acc = fmaf(wa.x, xv[0], acc);
            acc = fmaf(wa.y, xv[1], acc);
            acc = fmaf(wa.z, xv[2], acc);
            acc = fmaf(wa.w, xv[3], acc);
            acc = fmaf(wb.x, xv[4], acc);
            acc = fmaf(wb.y, xv[5], acc);
            acc = fmaf(wb.z, xv[6], acc);
            acc = fmaf(wb.w, xv[7], acc);
        }
        for (; k < k1; ++k) acc = fmaf(wr[k], xs[k * HW], acc);
    } else {
        // weight of (m, k): w[m*K + k], or w[k*M + m] with TRANS
        const int64_t wstep = TRANS ? M : 1;
        const float* wp = TRANS ? w + m : w + (int64_t)m * K;
        for (; k + 8 <= k1; k += 8) {
            float wv[8], xv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                wv[u] = wp[(k + u) * wstep];
                xv[u] = xs[(k + u) * HW];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = fmaf(wv[u], xv[u], acc);
        }
        for (; k < k1; ++k) acc = fmaf(wp[k * wstep], xs[k * HW], acc);
    }
    if (S == 1) {
        if (live) {
            float* zo = z + n * (int64_t)MH + o;
            if (ACC)
                *zo = *zo + acc;
            else
                *zo = BIAS ? bias[m] + acc : acc;
        }
        return;
    }
    part[v][lane] = acc;
    __syncthreads();
    if (v == 0 && live) {
        float t = part[0][lane];
        for (int i = 1; i < S; ++i) t += part[i][lane];
        float* zo = z + n * (int64_t)MH + o;
        if (ACC)
            *zo = *zo + t;
        else
            *zo = BIAS ? bias[m] + t : t;
    }
}

template <bool TRANS, bool V4, bool ACC, bool BIAS>
__global__ __launch_bounds__(1024) void k_pw_small(const float* __restrict__ x,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ z, int M, int K, int HW,
                                                   int seg) {
    __shared__ float part[kSmallMaxWaves][64];
    pw_small_body<TRANS, V4, ACC, BIAS>(x, w, bias, z, M, K, HW, seg, blockIdx.x, blockIdx.y,
                                        part);
}

// The same product for few input rows (K <= 64) over many pixels: a
// thread per pixel loads its K inputs once and forms CT outputs from them
// (k_pw_small gives every output its own thread, so each input is read M
// times through the caches: 16 -> 16 channels at 256^2 pixels read 64 MB
// for 4 MB of input).  Each output adds its K terms in k_pw_small's order
// with one wave per block row (k = 0, 1, ..., fmaf from zero, then the
// bias or the old value), so for K <= 32 the values are k_pw_small's.
constexpr int kPxCT = 16;  // outputs per thread

// K (the input rows) a template argument so the loops carry no bounds
// tests; the block's CT x K weights staged in LDS (each read is one
// address for the whole wave).
template <int K, bool TRANS, bool ACC, bool BIAS>
__global__ __launch_bounds__(256) void k_pw_px(const float* __restrict__ x,
                                               const float* __restrict__ w,
                                               const float* __restrict__ bias,
                                               float* __restrict__ z, int M, int HW) {
    __shared__ __attribute__((aligned(16))) float sw[kPxCT][K];
    const int p = (int)blockIdx.x * 256 + (int)threadIdx.x;
    const int64_t n = blockIdx.z;
    const int m0 = (int)blockIdx.y * kPxCT;
    const int jn = min(kPxCT, M - m0);  // block-uniform
    for (int i = threadIdx.x; i < kPxCT * K; i += 256) {
        const int j = i / K, k = i - j * K;
        sw[j][k] = j < jn ? (TRANS ? w[(int64_t)k * M + m0 + j] : w[(int64_t)(m0 + j) * K + k])
                          : 0.0f;
    }
    float xv[K];
    if (p < HW) {
        const float* xs = x + n * (int64_t)K * HW + p;
#pragma unroll
        for (int k = 0; k < K; ++k) xv[k] = xs[(int64_t)k * HW];
    }
    __syncthreads();
    if (p >= HW) return;
    float* zs = z + n * (int64_t)M * HW + p;
    for (int j = 0; j < jn; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(sw[j][k], xv[k], acc);
        const int m = m0 + j;
        float* zo = zs + (int64_t)m * HW;
        if (ACC)
            *zo = *zo + acc;
        else
            *zo = BIAS ? bias[m] + acc : acc;
    }
}

// K values with a k_pw_px instance
inline bool pw_px_k(int64_t K) {
    return K == 4 || K == 8 || K == 16 || K == 24 || K == 32 || K == 64;
}

// dW[co][ci] += sum_(n,p) dz[n][co][p] x[n][ci][p], db[co] += sum_(n,p)
// dz[n][co][p] for small planes.  Entry e (weights ci-fastest, then the
// C_out bias entries from E = C_out*C_in on) belongs to T = 2^lgT
// consecutive lanes; lane t sums the flattened (n, p) range [t*seg,
// (t+1)*seg) in float64, and the T partial sums meet in a fixed xor tree.
// A wave's x loads are consecutive pixels of consecutive rows; dz loads of
// one entry are shared by its lanes.  The grid covers entries [e0, e1)
// (e0 = E when only db is wanted).  V4: HW % 4 == 0, seg % 4 == 0 and
// 16-byte aligned dz and x.
// The body for flat lane `tid` (any block size that is a multiple of 64:
// the T lanes of an entry stay inside one wave).
template <bool V4>
__device__ __forceinline__ void pw_wgrad_small_body(const float* __restrict__ dz,
                                                    const float* __restrict__ x,
                                                    float* __restrict__ dw,
                                                    float* __restrict__ db, int N, int C_in,
                                                    int C_out, int HW, int64_t e0, int64_t e1,
                                                    int lgT, int seg, int64_t tid) {
    constexpr int W = V4 ? 4 : 1;  // pixels per load
    constexpr int U = 4;           // loads in flight per operand
    const int t = (int)(tid & ((1 << lgT) - 1));
    const int64_t e = e0 + (tid >> lgT);
    const bool valid = e < e1;
    const int64_t E = (int64_t)C_out * C_in;
    const int64_t ec = valid ? e : e1 - 1;
    const bool wt = ec < E;
    const int co = wt ? (int)(ec / C_in) : (int)(ec - E);
    const int ci = wt ? (int)(ec - (int64_t)co * C_in) : 0;
    const int64_t total = (int64_t)N * HW;
    int64_t q = (int64_t)t * seg;
    const int64_t qe = min(total, q + seg);
    double acc = 0.0;
    if (q < qe) {
        const int n0 = (int)(q / HW);
        int p = (int)(q - (int64_t)n0 * HW);
        const float* a = dz + ((int64_t)n0 * C_out + co) * HW;
        const float* b = x + ((int64_t)n0 * C_in + ci) * HW;
        const int64_t astep = (int64_t)C_out * HW, bstep = (int64_t)C_in * HW;
        auto fetch = [&](float (&av)[W], float (&bv)[W]) {
            if (V4) {
                const float4 u = *reinterpret_cast<const float4*>(a + p);
                av[0] = u.x, av[1] = u.y, av[2] = u.z, av[3] = u.w;
                if (wt) {
                    const float4 v = *reinterpret_cast<const float4*>(b + p);
                    bv[0] = v.x, bv[1] = v.y, bv[2] = v.z, bv[3] = v.w;
                }
            } else {
                av[0] = a[p];
                if (wt) bv[0] = b[p];
            }
            // next position: wrap to the following sample's plane
            p += W;
            const bool wrap = p == HW;
            p = wrap ? 0 : p;
            a = wrap ? a + astep : a;
            b = wrap ? b + bstep : b;
        };
        auto add = [&](const float (&av)[W], const float (&bv)[W]) {
#pragma unroll
            for (int i = 0; i < W; ++i) acc += wt ? (double)av[i] * (double)bv[i] : (double)av[i];
        };
        for (; q + U * W <= qe; q += U * W) {
            float av[U][W], bv[U][W];
#pragma unroll
            for (int u = 0; u < U; ++u) fetch(av[u], bv[u]);
#pragma unroll
            for (int u = 0; u < U; ++u) add(av[u], bv[u]);
        }
        for (; q < qe; q += W) {
            float av[W], bv[W];
            fetch(av, bv);
            add(av, bv);
        }
    }
    for (int off = (1 << lgT) >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (valid && t == 0) {
        float* out = wt ? dw + ec : db + co;
        *out = (float)((double)*out + acc);
    }
}

template <bool V4>
__global__ __launch_bounds__(256) void k_pw_wgrad_small(const float* __restrict__ dz,
                                                        const float* __restrict__ x,
                                                        float* __restrict__ dw,
                                                        float* __restrict__ db, int N, int C_in,
                                                        int C_out, int HW, int64_t e0,
                                                        int64_t e1, int lgT, int seg) {
    pw_wgrad_small_body<V4>(dz, x, dw, db, N, C_in, C_out, HW, e0, e1, lgT, seg,
                            (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// dx (+)= W^T dz and dW / db += the weight gradient of a small convolution
// in one launch (the two are independent and each is a few microseconds of
// mostly fixed cost): blocks [0, nbd) run k_pw_small's dx body over nbx
// output groups per sample, the others k_pw_wgrad_small's body on flat
// lanes.  Every output gets the same operations in the same order as from
// the two kernels.
template <bool ACC, bool V4W>
__global__ __launch_bounds__(1024) void k_pw_small_bwd(
    const float* __restrict__ dz, const float* __restrict__ w, float* __restrict__ dx,
    const float* __restrict__ x, float* __restrict__ dw, float* __restrict__ db, int N,
    int C_in, int C_out, int HW, int seg_d, int64_t nbx, int64_t nbd, int64_t e0, int64_t e1,
    int lgT, int seg_w) {
    __shared__ float part[kSmallMaxWaves][64];
    const int64_t b = blockIdx.x;
    if (b < nbd) {
        const int64_t n = b / nbx;
        pw_small_body<true, false, ACC, false>(dz, w, nullptr, dx, C_in, C_out, HW, seg_d,
                                               b - n * nbx, n, part);
    } else {
        pw_wgrad_small_body<V4W>(dz, x, dw, db, N, C_in, C_out, HW, e0, e1, lgT, seg_w,
                                 (b - nbd) * (int64_t)blockDim.x + threadIdx.x);
    }
}

template <typename F>
void bsel(bool b, F&& f) {
    if (b)
        f(std::true_type{});
    else
        f(std::false_type{});
}

}  // namespace

int pw_kpad(int64_t C_in) { return (int)((C_in + 7) / 8 * 8); }

bool pw_offsets_fit(int64_t C_in, int64_t HW) {
    // lane byte offsets (at most 20*HW for x and z, 256*C for w) stay below
    // 2^31: the buffer descriptors' range is 0x7fffffff bytes
    return HW <= ((int64_t)1 << 31) / 20 - 4 && C_in <= ((int64_t)1 << 31) / 256;
}

int64_t pw_pick_chunk(int64_t N, int64_t C_out, int64_t HW, int64_t max_chunk) {
    // enough waves to fill the chip (about 2048, two per SIMD): when the
    // planes are small, smaller chunks, down to one 128-pixel item
    const int64_t R = (C_out + kRowTile - 1) / kRowTile;
    const int64_t want = (2048 + N * R - 1) / std::max<int64_t>(N * R, 1);  // chunks per plane
    int64_t c = (HW + want - 1) / want;
    c = (c + kItem - 1) / kItem * kItem;
    return std::max<int64_t>(kItem, std::min<int64_t>(c, max_chunk));
}

namespace {
bool pw_small_fits(int64_t N, int64_t M, int64_t K, int64_t HW) {
    const int64_t lim = (int64_t)1 << 31;
    return N <= 65535 && M * HW < lim && K * HW < lim && M < lim && K < lim;
}

// Weight gradient on the SIMT kernel: at most small/2 multiply-adds, and
// at most 16384 (n, p) terms per entry (at most 256 per lane with 64 lanes
// per entry: a lane's sum is a chain of dependent loads).  Measured on
// MI355X (one sample, single launches): the SIMT kernel wins up to about
// 2^24 multiply-adds (e.g. 64x128 channels at 2048 pixels: 24 vs 30 us),
// the MFMA tiles from about 2^25 on; 16x4 channels at 262144 pixels (2^24
// multiply-adds, 4096 terms per lane) took 238 us against 25.
bool pw_use_small_wgrad(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t small) {
    return small > 0 && N * HW <= 16384 &&
           (double)N * (double)HW * (double)C_in * (double)C_out <= 0.25 * (double)small &&
           pw_small_fits(N, C_out, C_in, HW);
}
}  // namespace

// Measured on MI355X against the split-K MFMA kernel (one sample, single
// launches): the SIMT kernel wins up to about 2^25 multiply-adds (256 ->
// 128 channels at 1024 pixels: 11 vs 19 us; 64 -> 128 at 4096: 10 vs 13
// us), ties at 2^26 and loses above (512 -> 256 at 1024: 34 vs 28 us; 128
// -> 256 at 4096: 35 vs 16 us).
bool pw_use_small(int64_t N, int64_t M, int64_t K, int64_t HW, int64_t small) {
    return small > 0 && pw_small_fits(N, M, K, HW) &&
           (double)N * (double)M * (double)K * (double)HW <= (double)small;
}

namespace {

// z = W x (+ bias), or z += W x; TRANS: z = W^T x.  M output rows, K input
// rows.  Each wave sums about 32 values of K.
// Waves per block (K split) and K per wave of the SIMT kernel.
// Planes of at least this many pixels take k_pw_px when it has K (at most
// 32: the same sums as k_pw_small's one-wave blocks); K = 64, which
// k_pw_small splits over two waves (other partial sums), from
// kPxMinHW64 pixels on.
constexpr int64_t kPxMinHW = 1024;
constexpr int64_t kPxMinHW64 = 65536;  // (64 -> 32 at 16384 pixels: 10.3 vs 11 us)

struct PwSmallSplit {
    int S = 1;
    int64_t seg = 0;
};
PwSmallSplit pw_small_split(int64_t K) {
    PwSmallSplit r;
    r.S = (int)std::min<int64_t>(kSmallMaxWaves, std::max<int64_t>(1, (K + 31) / 32));
    r.seg = (K + r.S - 1) / r.S;
    r.seg = (r.seg + 3) / 4 * 4;
    r.S = (int)((K + r.seg - 1) / r.seg);
    return r;
}

// Lanes of the SIMT weight gradient: entries [e0, e1) (dW then db), 2^lgT
// lanes per entry over segments of `seg` pixels, about 64K lanes in all.
struct PwWgSmallPlan {
    int64_t e0 = 0, e1 = 0, lanes = 0;
    int lgT = 0;
    int64_t seg = 0;
    bool v4 = false;
};
PwWgSmallPlan pw_wgrad_small_plan(const float* dz, const float* x, bool want_dw, bool want_db,
                                  int64_t N, int64_t C_in, int64_t C_out, int64_t HW) {
    PwWgSmallPlan p;
    const int64_t E = C_out * C_in;
    p.e0 = want_dw ? 0 : E;
    p.e1 = want_db ? E + C_out : E;
    p.v4 = (HW % 4 == 0) && ((uintptr_t)dz % 16 == 0) && ((uintptr_t)x % 16 == 0);
    // segments of >= 8 pixels
    const int64_t nhw = N * HW, ne = p.e1 - p.e0;
    while (p.lgT < 6 && (ne << p.lgT) < 65536 && nhw > ((int64_t)8 << p.lgT)) ++p.lgT;
    p.seg = (nhw + (1 << p.lgT) - 1) >> p.lgT;
    if (p.v4) p.seg = (p.seg + 3) / 4 * 4;
    p.lanes = ne << p.lgT;
    return p;
}

hipError_t launch_pw_small(const float* x, const float* w, const float* bias, float* z,
                           int64_t N, int64_t K, int64_t M, int64_t HW, bool trans,
                           bool accumulate, hipStream_t s, const char* name) {
    const PwSmallSplit sp = pw_small_split(K);
    const int S = sp.S;
    const int64_t seg = sp.seg;
    const bool v4 = !trans && K % 4 == 0 && (uintptr_t)w % 16 == 0;
    const dim3 grid((unsigned)((M * HW + 63) / 64), (unsigned)N);
    const int tok = prof_begin(s, name);
    if (pw_px_k(K) && HW >= kPxMinHW && (S == 1 || HW >= kPxMinHW64)) {
        // few input rows over many pixels: a thread per pixel
        const dim3 pg((unsigned)((HW + 255) / 256), (unsigned)((M + kPxCT - 1) / kPxCT),
                      (unsigned)N);
        auto px = [&](auto T, auto A, auto B) {
            auto run = [&](auto KC) {
                k_pw_px<decltype(KC)::value, T(), A(), B()>
                    <<<pg, 256, 0, s>>>(x, w, bias, z, (int)M, (int)HW);
            };
            if (K == 4)
                run(std::integral_constant<int, 4>{});
            else if (K == 8)
                run(std::integral_constant<int, 8>{});
            else if (K == 64)
                run(std::integral_constant<int, 64>{});
            else if (K == 16)
                run(std::integral_constant<int, 16>{});
            else if (K == 24)
                run(std::integral_constant<int, 24>{});
            else
                run(std::integral_constant<int, 32>{});
        };
        using F = std::false_type;
        bsel(trans, [&](auto T) {
            if (accumulate)
                px(T, std::true_type{}, F{});
            else
                bsel(bias != nullptr, [&](auto B) { px(T, F{}, B); });
        });
        prof_end(s, tok);
        return hipGetLastError();
    }
    auto go = [&](auto T, auto V, auto A, auto B) {
        k_pw_small<T(), V(), A(), B()><<<grid, 64 * S, 0, s>>>(x, w, bias, z, (int)M, (int)K,
                                                               (int)HW, (int)seg);
    };
    using F = std::false_type;
    using Tr = std::true_type;
    if (trans) {
        bsel(accumulate, [&](auto A) { go(Tr{}, F{}, A, F{}); });
    } else {
        bsel(v4, [&](auto V) {
            if (accumulate)
                go(F{}, V, Tr{}, F{});
            else
                bsel(bias != nullptr, [&](auto B) { go(F{}, V, F{}, B); });
        });
    }
    prof_end(s, tok);
    return hipGetLastError();
}

}  // namespace

PwKz pw_kz_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t chunk,
                int kz_max) {
    PwKz r;
    if (kz_max < 2 || N == 0 || HW == 0 || C_out == 0 || N > 65535) return r;
    const int64_t cpp = (HW + chunk - 1) / chunk;
    const int64_t R = (C_out + kRowTile - 1) / kRowTile;
    const int64_t groups = (R + kRowGroup - 1) / kRowGroup;
    const int64_t rpw = N * cpp * groups >= 1024 ? kRowGroup : 1;
    const int64_t tiles = N * cpp * ((R + rpw - 1) / rpw);
    const int64_t ksteps = pw_kpad(C_in) / 8;
    // (K of 128 measured slower split: 128 -> 256 channels at 4096 pixels,
    // 31.5 us per fused forward in-block, 33 us over blocks)
    if (tiles >= kKzTiles || ksteps < 32) return r;
    // four waves per block (one CU), blocks for about 2048 waves in all,
    // at least two K steps per wave
    int kz = 1;
    while (2 * kz <= kz_max && tiles * 4 * (2 * kz) <= 2048 && ksteps >= kKzStepsPerWave * 4 * (2 * kz)) kz *= 2;
    if (kz > 1) r.kz = kz;
    return r;
}

size_t pw_kz_bytes(int64_t N, int64_t C_out, int64_t HW, int kz) {
    if (kz < 2) return 0;
    return ((size_t)kz * (size_t)(N * C_out * HW) * sizeof(float) + 255) & ~(size_t)255;
}

size_t pw_kz_max_bytes(int64_t N, int64_t C_out, int64_t HW, int64_t chunk, int kz_max) {
    // the largest C_in: any K big enough for kz_max
    return pw_kz_bytes(N, C_out, HW, pw_kz_plan(N, (int64_t)1 << 20, C_out, HW, chunk, kz_max).kz);
}

namespace {
// Small grids: KZ blocks per output tile, each taking a K segment with four
// waves, write fp32 slices; k_pw_kz_reduce adds them (with the bias, the
// old z, the GroupNorm partials).  Deterministic: fixed segments, slices
// added in order.
hipError_t launch_pw_kz(const PwArgs& a, int64_t N, int64_t C_in, int64_t C_out, int64_t HW,
                        int64_t chunk, double2* part, bool accumulate, int kz, float* ws,
                        hipStream_t s) {
    const int64_t cpp = (HW + chunk - 1) / chunk;
    const int64_t R = (C_out + kRowTile - 1) / kRowTile;
    const int64_t groups = (R + kRowGroup - 1) / kRowGroup;
    const int rpw = N * cpp * groups >= 1024 ? kRowGroup : 1;
    const dim3 grid((unsigned)(N * cpp), (unsigned)((R + rpw - 1) / rpw), (unsigned)kz);
    const bool fast = (HW % 4 == 0) && (C_in % 8 == 0) && ((uintptr_t)a.x % 16 == 0) &&
                      ((uintptr_t)ws % 16 == 0) && ((uintptr_t)a.w % 16 == 0);
    const int Kpad = pw_kpad(C_in), ksteps = Kpad / 8;
    const int kzsteps = (ksteps + kz - 1) / kz;
    const int kzseg = kzsteps * 8, kseg = (kzsteps + 3) / 4 * 8;
    const int64_t zslice = N * C_out * HW;
    bsel(fast, [&](auto F) {
        k_pw_conv<F(), kPlain, false, 4, 1><<<grid, 256, 0, s>>>(
            a.x, a.w, nullptr, ws, nullptr, C_in, C_out, HW, chunk, cpp, Kpad, rpw, kseg,
            kzseg, zslice);
    });
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool v4 = HW % 4 == 0 && (uintptr_t)a.z % 16 == 0 && (uintptr_t)ws % 16 == 0;
    const dim3 rg((unsigned)cpp, (unsigned)((C_out + 3) / 4), (unsigned)N);
    auto run = [&](auto ST, auto B, auto A) {
        bsel(v4, [&](auto V) {
            k_pw_kz_reduce<ST(), B(), A(), V()><<<rg, 256, 0, s>>>(ws, a.bias, a.z, part, kz,
                                                                   zslice, C_out, HW, chunk, cpp);
        });
    };
    // (launch_pw_conv splits over blocks only with the statistics; the
    // kernel's plain and accumulate forms are kept for reuse)
    (void)accumulate;
    bsel(a.bias != nullptr, [&](auto B) { run(std::true_type{}, B, std::false_type{}); });
    return hipGetLastError();
}
}  // namespace

hipError_t launch_pw_conv(const PwArgs& a, int64_t N, int64_t C_in, int64_t C_out,
                          int64_t HW, int64_t chunk, double2* part, bool accumulate,
                          int64_t small, float* kz_ws, int kz_max, hipStream_t s,
                          const char* name, bool wt) {
    if (N == 0 || HW == 0 || C_out == 0) return hipSuccess;
    if (!part && pw_use_small(N, C_out, C_in, HW, small))
        return launch_pw_small(a.x, a.w, a.bias, a.z, N, C_in, C_out, HW, false, accumulate, s,
                               name ? name : "pw_conv_small");
    if (kz_ws && part) {
        const PwKz kp = pw_kz_plan(N, C_in, C_out, HW, chunk, kz_max);
        if (kp.kz > 1) {
            if (!name) name = part ? "pw_conv_gn_stats" : "pw_conv";
            const int tok = prof_begin(s, name);
            const hipError_t e =
                launch_pw_kz(a, N, C_in, C_out, HW, chunk, part, accumulate, kp.kz, kz_ws, s);
            prof_end(s, tok);
            return e;
        }
    }
    const int64_t cpp = (HW + chunk - 1) / chunk;
    // A wave walks up to kRowGroup row tiles of its chunk (the chunk's x
    // stays in cache across them); when that leaves too few waves, each row
    // tile gets its own wave.
    const int64_t R = (C_out + kRowTile - 1) / kRowTile;
    const int64_t groups = (R + kRowGroup - 1) / kRowGroup;
    const int rpw = N * cpp * groups >= 1024 ? kRowGroup : 1;
    const dim3 grid((unsigned)(N * cpp), (unsigned)((R + rpw - 1) / rpw));
    const bool fast = (HW % 4 == 0) && (C_in % 8 == 0) && ((uintptr_t)a.x % 16 == 0) &&
                      ((uintptr_t)a.z % 16 == 0) && ((uintptr_t)a.w % 16 == 0);
    const int Kpad = pw_kpad(C_in);
    const int mode = part ? kStats : (accumulate ? kAccum : kPlain);
    if (!name) name = part ? "pw_conv_gn_stats" : "pw_conv";
    // Split K over 2 or 4 waves of a block while the grid stays within
    // 2048 waves and each wave keeps at least 4 K steps: a wave's time is
    // its K/8 dependent MFMA steps, so a small grid finishes sooner.
    const int64_t waves = (int64_t)grid.x * grid.y, ksteps = Kpad / 8;
    int ks = 1;
    while (ks < 4 && waves * ks * 2 <= 2048 && ksteps >= 8 * ks) ks *= 2;
    const int kseg = (int)((ksteps + ks - 1) / ks) * 8;
    const int tok = prof_begin(s, name);
    // Large grids of the fast path run one wave per SIMD with two K steps
    // in flight (the accumulators then fit in AGPRs with no spills; at
    // 64 -> 64 channels over 2048^2 pixels the statistics variant took 483
    // instead of 556 us, the plain one 456 instead of 469); split-K and the
    // general path keep two waves per SIMD and one step in flight.
    // The streamed kernel (kSd steps in flight across items) when the K
    // steps fill its operand ring exactly: the statistics variant at
    // 64 -> 64 channels over 2048^2 pixels took 484-489 us instead of
    // 505-512 us.
    const bool stream = fast && ks == 1 && ksteps % (kSd + 1) == 0;
    auto go = [&](auto F, auto M, auto B) {
        if constexpr (F()) {
            if (stream) {
                k_pw_conv_stream<M(), B()><<<grid, 64, 0, s>>>(a.x, a.w, a.bias, a.z, part, C_in,
                                                              C_out, HW, chunk, cpp, Kpad, rpw);
                return;
            }
        }
        auto run = [&](auto K, auto D) {
            k_pw_conv<F(), M(), B(), K(), D()><<<grid, 64 * K(), 0, s>>>(
                a.x, a.w, a.bias, a.z, part, C_in, C_out, HW, chunk, cpp, Kpad, rpw, kseg, Kpad,
                0);
        };
        using D1 = std::integral_constant<int, 1>;
        if (ks == 4)
            run(std::integral_constant<int, 4>{}, D1{});
        else if (ks == 2)
            run(std::integral_constant<int, 2>{}, D1{});
        else if constexpr (F())
            run(D1{}, std::integral_constant<int, 2>{});
        else
            run(D1{}, D1{});
    };
    using P = std::integral_constant<int, kPlain>;
    using S = std::integral_constant<int, kStats>;
    using A = std::integral_constant<int, kAccum>;
    bsel(fast, [&](auto F) {
        if (wt) {  // transposed weights: dx = W^T dz, no bias, no statistics
            if (mode == kAccum)
                go(F, std::integral_constant<int, kAccumT>{}, std::false_type{});
            else
                go(F, std::integral_constant<int, kPlainT>{}, std::false_type{});
        } else if (mode == kAccum) {
            go(F, A{}, std::false_type{});
        } else {
            bsel(a.bias != nullptr, [&](auto B) {
                if (mode == kStats)
                    go(F, S{}, B);
                else
                    go(F, P{}, B);
            });
        }
    });
    prof_end(s, tok);
    return hipGetLastError();
}

PwBwdPlan make_pw_bwd_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW,
                           int64_t chunk_dx, int kz_max, int wg_waves, int64_t wg_target) {
    PwBwdPlan p;
    // dx = W^T dz: M = C_in outputs, K = C_out terms.  (Its split-K over
    // blocks measured no gain: a plain 256 -> 128 output at 4096 pixels took
    // 18.6 us with K over the four waves of a block, 14.3 + 4.2 us as four
    // blocks' slices plus their reduce.  The statistics variant gains.)
    p.chunk_dx = pw_pick_chunk(N, C_in, HW, chunk_dx);
    p.kz_dx = pw_kz_plan(N, C_out, C_in, HW, p.chunk_dx, std::min(kz_max, 1)).kz;
    p.kz_bytes = pw_kz_bytes(N, C_in, HW, p.kz_dx);
    p.tm = C_out <= 32 ? 1 : 2;
    p.tn = C_in <= 32 ? 1 : 2;
    p.tiles_co = (C_out + 32 * p.tm - 1) / (32 * p.tm);
    p.tiles_ci = (C_in + 32 * p.tn - 1) / (32 * p.tn);
    // about 2048 waves (two per SIMD), chunks of at least 64 pixels (a wave
    // spends about 1.7 us per 32-pixel step on its 64x64 tile, so small
    // grids get short chunks; each chunk adds a partial tile to the finish)
    const int64_t total = N * HW * p.tiles_co * p.tiles_ci;
    int64_t chunk = (total / wg_target + 31) / 32 * 32;
    chunk = std::max<int64_t>(chunk, 64);
    const int64_t hw32 = (HW + 31) / 32 * 32;
    p.chunk = std::min(chunk, std::max<int64_t>(hw32, 32));
    p.cpp = (HW + p.chunk - 1) / p.chunk;
    p.G = N * p.cpp;
    // waves per block (a power of two, each with at least one step of a
    // plane) on chunks of wpb wave chunks; the partials are sized for one
    // per wave chunk, which covers any wpb
    p.wpb = 1;
    while (p.wpb < wg_waves && 2 * p.wpb <= p.G && 2 * p.wpb * kWgStep <= hw32) p.wpb *= 2;
    p.chunk_b = std::min(p.chunk * p.wpb, hw32);
    p.cpp_b = (HW + p.chunk_b - 1) / p.chunk_b;
    p.Gb = N * p.cpp_b;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    p.wt_bytes = al(sizeof(float) * (size_t)(C_in * C_out));
    p.pw_bytes = al(sizeof(float) * (size_t)(p.G * C_out * C_in));
    p.pb_bytes = al(sizeof(float) * (size_t)(p.G * C_out));
    return p;
}

size_t pw_bwd_workspace_bytes(const PwBwdPlan& p) {
    return p.wt_bytes + p.pw_bytes + p.pb_bytes + p.kz_bytes;
}

hipError_t launch_pw_backward(const PwBwdPlan& p, const PwBwdArgs& a, int64_t N, int64_t C_in,
                              int64_t C_out, int64_t HW, bool accumulate_dx, int64_t small,
                              hipStream_t s) {
    if (N == 0 || HW == 0 || C_out == 0 || C_in == 0) return hipSuccess;
    char* ws = static_cast<char*>(a.ws);
    float* wt = reinterpret_cast<float*>(ws);
    float* part_w = reinterpret_cast<float*>(ws + p.wt_bytes);
    float* part_b = reinterpret_cast<float*>(ws + p.wt_bytes + p.pw_bytes);
    const bool small_dx = a.dx && pw_use_small(N, C_in, C_out, HW, small);
    const bool small_dw = (a.dw || a.db) && pw_use_small_wgrad(N, C_in, C_out, HW, small);
    if (small_dx && small_dw) {
        // both SIMT kernels in one launch, on dx's block shape
        const PwSmallSplit sp = pw_small_split(C_out);
        const PwWgSmallPlan wp = pw_wgrad_small_plan(a.dz, a.x, a.dw, a.db, N, C_in, C_out, HW);
        const int64_t threads = 64 * (int64_t)sp.S;
        const int64_t nbx = (C_in * HW + 63) / 64, nbd = nbx * N;
        const int64_t nbw = (wp.lanes + threads - 1) / threads;
        const int tok = prof_begin(s, "pw_conv_bwd_small");
        bsel(accumulate_dx, [&](auto A) {
            bsel(wp.v4, [&](auto V) {
                k_pw_small_bwd<A(), V()><<<dim3((unsigned)(nbd + nbw)), (unsigned)threads, 0, s>>>(
                    a.dz, a.w, a.dx, a.x, a.dw, a.db, (int)N, (int)C_in, (int)C_out, (int)HW,
                    (int)sp.seg, nbx, nbd, wp.e0, wp.e1, wp.lgT, (int)wp.seg);
            });
        });
        prof_end(s, tok);
        return hipGetLastError();
    }
    if (small_dx) {
        // dx = W^T dz, reading W transposed in place
        hipError_t e = launch_pw_small(a.dz, a.w, nullptr, a.dx, N, C_out, C_in, HW, true,
                                       accumulate_dx, s, "pw_conv_dgrad_small");
        if (e != hipSuccess) return e;
    } else if (a.dx) {
        // dx = W^T dz: the forward kernel with dz as input and W^T as
        // weights.  Small grids read W in place (transposed-weight modes:
        // no transpose launch, which costs them more than the extra
        // loads); large grids transpose W into the workspace first.
        const int64_t cpp = (HW + p.chunk_dx - 1) / p.chunk_dx;
        const int64_t R = (C_in + kRowTile - 1) / kRowTile;
        const bool in_place = N * cpp * R < kKzTiles;
        if (!in_place) {
            const int64_t E = C_in * C_out;
            int tok = prof_begin(s, "pw_transpose");
            k_transpose<<<dim3((unsigned)((E + 255) / 256)), 256, 0, s>>>(a.w, wt, C_out, C_in);
            prof_end(s, tok);
        }
        PwArgs fa{a.dz, in_place ? a.w : wt, nullptr, a.dx};
        float* kz_ws = p.kz_dx > 1 ? reinterpret_cast<float*>(ws + p.wt_bytes + p.pw_bytes +
                                                               p.pb_bytes)
                                   : nullptr;
        hipError_t e = launch_pw_conv(fa, N, C_out, C_in, HW, p.chunk_dx, nullptr,
                                      accumulate_dx, 0, kz_ws, p.kz_dx, s, "pw_conv_dgrad",
                                      in_place);
        if (e != hipSuccess) return e;
    }
    if (small_dw) {
        const PwWgSmallPlan wp = pw_wgrad_small_plan(a.dz, a.x, a.dw, a.db, N, C_in, C_out, HW);
        const int tok = prof_begin(s, "pw_conv_wgrad_small");
        bsel(wp.v4, [&](auto V) {
            k_pw_wgrad_small<V()><<<dim3((unsigned)((wp.lanes + 255) / 256)), 256, 0, s>>>(
                a.dz, a.x, a.dw, a.db, (int)N, (int)C_in, (int)C_out, (int)HW, wp.e0, wp.e1,
                wp.lgT, (int)wp.seg);
        });
        prof_end(s, tok);
    } else if (a.dw || a.db) {
        const bool fast = (HW % 4 == 0) && ((uintptr_t)a.dz % 16 == 0) &&
                          ((uintptr_t)a.x % 16 == 0);
        const dim3 grid((unsigned)(p.tiles_co * p.tiles_ci), (unsigned)p.Gb);
        int tok = prof_begin(s, "pw_conv_wgrad");
        auto launch = [&](auto F, auto M2, auto N2, auto W) {
            k_pw_wgrad<F(), M2() ? 2 : 1, N2() ? 2 : 1, W()><<<grid, 64 * W(), 0, s>>>(
                a.dz, a.x, part_w, part_b, C_in, C_out, HW, p.chunk_b, p.cpp_b, p.tiles_ci);
        };
        bsel(fast, [&](auto F) {
            bsel(p.tm == 2, [&](auto M2) {
                bsel(p.tn == 2, [&](auto N2) {
                    switch (p.wpb) {
                        case 1: launch(F, M2, N2, std::integral_constant<int, 1>{}); break;
                        case 2: launch(F, M2, N2, std::integral_constant<int, 2>{}); break;
                        case 4: launch(F, M2, N2, std::integral_constant<int, 4>{}); break;
                        default: launch(F, M2, N2, std::integral_constant<int, 8>{}); break;
                    }
                });
            });
        });
        prof_end(s, tok);
        const int64_t E = C_out * C_in;
        if (weight_finish_deferring()) {  // queued for the model's one finish launch
            hipError_t qe = hipSuccess;
            if (a.dw) weight_finish_queue({part_w, a.dw, nullptr, E, p.Gb, 0}, s, &qe);
            if (qe == hipSuccess && a.db)
                weight_finish_queue({part_b, a.db, nullptr, C_out, p.Gb, 0}, s, &qe);
            if (qe != hipSuccess) return qe;
            return hipGetLastError();
        }
        tok = prof_begin(s, "pw_conv_wgrad_finish");
        // dW and db in one launch
        const int64_t nbw = a.dw ? (E + 63) / 64 : 0, nbb = a.db ? (C_out + 63) / 64 : 0;
        k_sum_partials<<<dim3((unsigned)(nbw + nbb)), 1024, 0, s>>>(part_w, a.dw, E, nbw, part_b,
                                                                    a.db, C_out, p.Gb);
        prof_end(s, tok);
    }
    return hipGetLastError();
}

bool pw_cba_fused_fits(int64_t C_in, int64_t C_out, int64_t HW) {
    // one dW tile; in-sample byte offsets (64 rows of HW floats) in 31 bits
    // and whole 8-row slots: C_in and C_out multiples of 8 (k_pw_cba_bwd's
    // loads and stores stay inside each sample's rows with scalar row offsets)
    return C_in >= 8 && C_in <= 64 && C_in % 8 == 0 && C_out >= 8 && C_out <= 64 &&
           C_out % 8 == 0 && HW >= 4 && HW % 4 == 0 &&
           HW <= ((int64_t)1 << 31) / 256 - 64;
}

PwCbaPlan make_pw_cba_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t target) {
    PwCbaPlan p;
    constexpr int64_t kStep = (int64_t)kWgStep * kFbPairs;  // pixels per block step
    const int64_t per = (N * HW + std::max<int64_t>(target, 1) - 1) / std::max<int64_t>(target, 1);
    int64_t chunk = (per + kStep - 1) / kStep * kStep;
    chunk = std::max(chunk, kStep);
    p.chunk = std::min(chunk, (HW + kStep - 1) / kStep * kStep);
    p.cpp = (HW + p.chunk - 1) / p.chunk;
    p.blocks = N * p.cpp;
    p.part_bytes = ((size_t)p.blocks * (size_t)(C_out * C_in) * sizeof(float) + 255) & ~(size_t)255;
    return p;
}

hipError_t launch_pw_cba_backward(const PwCbaPlan& p, const PwCbaArgs& a, int64_t N,
                                  int64_t C_in, int64_t C_out, int64_t HW, int64_t G, bool silu,
                                  bool accumulate_dx, hipStream_t s) {
    if (N == 0 || HW == 0) return hipSuccess;
    const int tm = C_out <= 32 ? 1 : 2, tn = C_in <= 32 ? 1 : 2;
    float* part = a.dw ? a.part_w : nullptr;
    int tok = prof_begin(s, "pw_cba_bwd");
    const bool full = C_out == 32 * tm && C_in == 32 * tn;
    auto go = [&](auto S, auto M2, auto N2, auto A, auto F) {
        k_pw_cba_bwd<S(), M2() ? 2 : 1, N2() ? 2 : 1, A(), F()>
            <<<dim3((unsigned)p.blocks), 128 * kFbPairs, 0, s>>>(
                a.dy, a.z, a.x, a.w, a.gamma, a.beta, a.mean, a.rstd, a.mean_lo, a.unit_sums,
                a.plane_sums, a.dgamma, a.dbeta, a.dx, part, C_in, C_out, HW, G, N, p.chunk,
                p.cpp, a.gn_part, a.gn_cpp);
    };
    bsel(silu, [&](auto S) {
        bsel(tm == 2, [&](auto M2) {
            bsel(tn == 2, [&](auto N2) {
                bsel(accumulate_dx, [&](auto A) { bsel(full, [&](auto F) { go(S, M2, N2, A, F); }); });
            });
        });
    });
    prof_end(s, tok);
    if (a.dw) {
        const int64_t E = C_out * C_in;
        hipError_t qe = hipSuccess;
        if (weight_finish_queue({part, a.dw, nullptr, E, p.blocks, 0}, s, &qe))
            return qe != hipSuccess ? qe : hipGetLastError();
        tok = prof_begin(s, "pw_cba_wgrad_finish");
        k_sum_partials<<<dim3((unsigned)((E + 63) / 64)), 1024, 0, s>>>(
            part, a.dw, E, (E + 63) / 64, nullptr, nullptr, 0, p.blocks);
        prof_end(s, tok);
    }
    return hipGetLastError();
}

}  // namespace gn
}  // namespace soar
