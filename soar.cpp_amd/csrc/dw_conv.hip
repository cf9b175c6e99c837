// dw_conv.hip - depthwise convolution (groups = C_in = C_out) forward and
// backward for gfx950: the K x K / stride / dilation convolutions of the
// CBA blocks Down.dw (k3 s2), LKR.dw (k5, k7) and the Ctx branches (k3 with
// dilation 1, 3, 5) of pomagrenate/soar.cpp (src/nn/blocks.cpp:449-500).
//
// Reference: src/cuda/ops/convolution_kernels.cu:138-333 (one thread per
// output reading every tap from global memory) and the CPU loops of
// src/nn/layers.cpp:400-428, 150-230.  Output size and zero padding follow
// Conv2d (layers.cpp:326-332): taps outside the input are skipped.
//
// Fast kernels (template K, S, D for the configurations the model uses):
// a 256-thread block owns a column of 32 x 64 output tiles (4, 8 at K = 5,
// 16 at K = 7: conv_per) of
// one (n, c) plane.  The input tile each needs, halo included, is staged in
// LDS from coalesced loads (zeros outside the image); the loads of the next
// tile go out into registers before the current tile is computed, so they
// are in flight during its FMAs (one tile per block waited on its loads
// about 80% of the time: 0.62 vs 0.47 ms for k3 at 64 x 2048^2).  Each
// thread then computes 8
// consecutive outputs of one row, reading each of the K input row segments
// it touches with 16-byte LDS loads into registers and applying all K
// taps of that row from registers.  Per output that is about K*(8S+(K-1)D)/8
// LDS floats instead of K*K, and the weights are wave-uniform scalars.
//   forward  y  = b + w (*) x
//   dx, S=1  dx (+)= flip(w) (*) dy with pad' = (K-1)*D - pad (the adjoint
//            of a stride-1 convolution is the convolution with the flipped
//            kernel), same kernel
//   dx, S>1  gather per input element over the taps that divide (as the
//            reference's k_conv2d_dw_backward_input), over a dy region
//            staged in LDS
//   dw, db   the block's K*K tap sums and its dy sum over its tile, reduced
//            in the block in a fixed order, written as per-tile partials and
//            added by a fixed-order float64 finish
// Other (K, S, D): generic kernels with the same results up to summation
// order.
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

constexpr int kTH = 32;       // output rows per tile
constexpr int kTW = 64;       // output columns per tile
constexpr int kPer = 8;       // consecutive outputs per thread
constexpr int kDwThreads = 256;

constexpr int round4(int v) { return (v + 3) / 4 * 4; }

// Input tile of a 32*RB x 64 output tile (RB output rows per thread).
template <int K, int S, int D, int RB = 1, bool SP = false>
struct Tile {
    static constexpr int TH = kTH * RB;                          // output rows
    static constexpr int IH = (TH - 1) * S + (K - 1) * D + 1;    // input rows
    static constexpr int IW = (kTW - 1) * S + (K - 1) * D + 1;   // input columns
    static constexpr int SL = (kPer - 1) * S + (K - 1) * D + 1;  // a thread's row segment
    static constexpr int SL4 = round4(SL);
    // row pitch: every thread's 16-byte segment reads stay inside the row
    static constexpr int IWP0 = round4(IW) > (kTW - kPer) * S + SL4 ? round4(IW)
                                                                    : (kTW - kPer) * S + SL4;
    // SP (stride 1, one row per thread): a pitch that spreads a read pass
    // over the LDS banks.  A 16-byte read is served 16 lanes at a time, two
    // eight-lane groups on consecutive rows; one row's eight segments start
    // 32 bytes apart.  Measured on a k7 tap window of reads (time per row
    // read), pitch 68 / 72 / 76 / 80 / 84 floats: 49 / 70 / 48 / 89 / 48,
    // so the pitch takes an odd number of 16-byte chunks (k7 and k3 at
    // dilation 3: 72 -> 76).  The kernels that read two tiles per step use
    // it (fused CBA backward k7 1.16 -> 1.10 ms, weight gradient 0.513 ->
    // 0.476 ms at 64 x 2048^2); the convolutions gain less than the padding
    // costs them (k7 0.542 -> 0.551 ms) and keep the plain pitch.
    static constexpr int pitch() {
        int p = IWP0;
        if (!SP || S != 1 || RB != 1) return p;
        while ((p / 4) % 2 == 0) p += 4;
        return p;
    }
    static constexpr int IWP = pitch();
    static constexpr int floats = IH * IWP;
};

// Row segment of a thread: SL4 floats of LDS row `lrow` from column c0*S.
template <int K, int S, int D, int RB = 1, bool SP = false>
__device__ __forceinline__ void load_seg(const float* tile, int lrow, int c0,
                                         float (&seg)[Tile<K, S, D, RB, SP>::SL4]) {
    using T = Tile<K, S, D, RB, SP>;
    const f4* p = reinterpret_cast<const f4*>(tile + lrow * T::IWP + c0 * S);
#pragma unroll
    for (int q = 0; q < T::SL4 / 4; ++q) {
        const f4 v = p[q];
        seg[4 * q] = v.x;
        seg[4 * q + 1] = v.y;
        seg[4 * q + 2] = v.z;
        seg[4 * q + 3] = v.w;
    }
}

// A thread's share of a tile's input (element i = threadIdx.x + k*256 of
// the LDS tile), fetched into registers so the loads of the next tile are
// in flight while the current one is computed.
template <int K, int S, int D, int RB = 1, bool SP = false>
struct TilePrefetch {
    static constexpr int NR = (Tile<K, S, D, RB, SP>::floats + kDwThreads - 1) / kDwThreads;
    float v[NR];

    // input rows [iy0, iy0 + IH) x columns [ix0, ix0 + IWP) of plane `ip`
    // (zeros outside the image and past column IW).  32-bit offsets: a
    // plane holds fewer than 2^31 elements (checked by the host).  The
    // element index is recomputed for every tile (not hoisted out of the
    // tile loop, where NR offsets would stay live in registers).
    // With lr0 > 0 only local rows [lr0, IH) are fetched (the rows above
    // come from the previous tile, see HaloRows).
    __device__ __forceinline__ void fetch(const float* __restrict__ ip, int iy0, int ix0, int Hi,
                                          int Wi, int lr0 = 0) {
        using T = Tile<K, S, D, RB, SP>;
        const int nel = (T::IH - lr0) * T::IWP, base = lr0 * T::IWP;
        int t = (int)threadIdx.x;
        asm volatile("" : "+v"(t));
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = t + k * kDwThreads;
            const int li = base + i;
            const int r = li / T::IWP, col = li - r * T::IWP;
            const int yy = iy0 + r, xx = ix0 + col;
            float x = 0.0f;
            if (i < nel && col < T::IW && (unsigned)yy < (unsigned)Hi &&
                (unsigned)xx < (unsigned)Wi)
                x = ip[yy * Wi + xx];
            v[k] = x;
        }
    }
    __device__ __forceinline__ void stash(float* tile, int lr0 = 0) const {
        using T = Tile<K, S, D, RB, SP>;
        const int nel = (T::IH - lr0) * T::IWP, base = lr0 * T::IWP;
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = (int)threadIdx.x + k * kDwThreads;
            if (i < nel) tile[base + i] = v[k];
        }
    }
};

// Word 3 of a raw buffer descriptor on gfx9-family parts (gfx950 included):
// 32-bit float data format, no swizzle, no stride.
constexpr int kRsrcWord3 = 0x00020000;

// Stride 1, every tile of a block after its first: the TH new rows
// [O, IH) of the haloed tile (the rows above move up from the previous
// tile, HaloRows), whose first is image row y > 0 (y = TH*(tile + 1) - pad
// + O with pad <= O).  A thread's elements (TilePrefetch's: element
// i = t + 256 k of those rows, row i / IWP, column i % IWP) lie at fixed
// byte offsets from row y, computed once per block.  A tile then loads
// through a buffer descriptor based at row y whose range ends at the
// plane's end: elements of rows past the bottom read zeros without a test,
// and columns outside the image or past IW carry an offset past any range,
// so they read zeros too.  Per element that leaves the load itself,
// against a division, bounds tests and a 64-bit address before.  Byte
// offsets within TH rows fit 31 bits (planes_fit_32).
// ROWS: rows fetched (TH: the new rows of a halo walk; IH: a whole tile,
// for walks that fetch every tile whole, whose later tiles start at image
// rows y > 0 as well).
template <int K, int D, int RB = 1, int ROWS = kTH * RB, bool SP = false>
struct HaloFetch {
    using T = Tile<K, 1, D, RB, SP>;
    static constexpr int NEL = ROWS * T::IWP;
    static constexpr int NF = (NEL + kDwThreads - 1) / kDwThreads;
    static constexpr uint32_t kOut = 0x80000000u;  // past any range
    uint32_t off[NF];
    __device__ __forceinline__ void init(int ix0, int Wi) {
        const int t = threadIdx.x;
#pragma unroll
        for (int k = 0; k < NF; ++k) {
            const int i = t + k * kDwThreads;
            const int r = i / T::IWP, col = i - r * T::IWP, xx = ix0 + col;
            const bool ok = i < NEL && col < T::IW && (unsigned)xx < (unsigned)Wi;
            off[k] = ok ? (uint32_t)(r * Wi + xx) * 4u : kOut;
        }
    }
    // range (bytes) of the rows from image row y to the plane's end
    __device__ __forceinline__ static int range(int y, int Hi, int Wi) {
        const int64_t rem = (int64_t)(Hi - y) * Wi * 4;
        return (int)(rem < 0 ? 0 : (rem > 0x7fffffff ? 0x7fffffff : rem));
    }
    __device__ __forceinline__ static auto rsrc(const float* ip, int y, int lim, int Wi) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ip + (int64_t)y * Wi), (short)0,
                                                 lim, kRsrcWord3);
    }
    template <typename R, int NR>
    __device__ __forceinline__ void load(const R& rs, float (&v)[NR]) const {
        static_assert(NF <= NR, "prefetch slots");
#pragma unroll
        for (int k = 0; k < NF; ++k)
            v[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off[k], 0, 0));
    }
};

// Stride 1: consecutive 32-row tiles of a block overlap in O = (K-1)*D
// input rows (local rows [kTH, kTH + O) of one are rows [0, O) of the
// next).  They move to the top of the LDS tile through NS registers per
// thread instead of being fetched again, so after its first tile a block
// fetches its kTH new rows only.
template <int K, int D, int RB = 1, bool SP = false>
struct HaloRows {
    using T = Tile<K, 1, D, RB, SP>;
    static constexpr int O = (K - 1) * D;
    static constexpr int NS = (O * T::IWP + kDwThreads - 1) / kDwThreads;
    float v[NS];
    // after the tile is in LDS (and before the next one is stashed)
    __device__ __forceinline__ void take(const float* tile) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int j = (int)threadIdx.x + k * kDwThreads;
            if (j < O * T::IWP) v[k] = tile[T::TH * T::IWP + j];
        }
    }
    // after every thread's reads of the previous tile are done
    __device__ __forceinline__ void put(float* tile) const {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const int j = (int)threadIdx.x + k * kDwThreads;
            if (j < O * T::IWP) tile[j] = v[k];
        }
    }
};

// out (+)= bias + w (*) in over `per` 32 x 64 output tiles down one plane
// per block (tile rows tyg*per ..): the input of tile i + 1 is fetched into
// registers while tile i is computed from LDS.  FLIP
// applies the kernel rotated by 180 degrees (the stride-1 input gradient).
// (body of block b; `tile` holds Tile<K, S, D>::floats floats)
// STATS (forward): the GroupNorm statistics epilogue.  Each thread sums its
// stored outputs shifted by its first one (a data value, so the sums stay
// small when |mean| >> std), and the block combines them into the (mean,
// M2) of its tile column, part[b] (block_moments, gn_moments.hpp).  Block b
// = plane * tpp + group, so a unit's partials lie together, plane-major:
// the layout the GroupNorm finish combines (with the tiles' element counts,
// dw_stats_geometry), so no statistics pass re-reads the output.
// `mom`: 4 * kDwThreads / 64 doubles of LDS.
template <int K, int S, int D, bool FLIP, bool ACC, bool BIAS, bool STATS = false>
__device__ __forceinline__ void dw_conv_body(
    const float* __restrict__ in, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo,
    int64_t pad, int64_t tiles_x, int64_t tiles_y, int64_t tpp, int per, int64_t b,
    float* __restrict__ tile, double2* __restrict__ part = nullptr, double* mom = nullptr) {
    using T = Tile<K, S, D>;
    const int64_t plane = b / tpp, gix = b - plane * tpp;
    const int64_t c = plane % C;
    const int64_t tyg = gix / tiles_x, tx = gix - tyg * tiles_x;
    const int64_t ty0 = tyg * per, ty1 = min(ty0 + per, tiles_y);
    const int64_t ox0 = tx * kTW;
    const float* ip = in + plane * Hi * Wi;
    TilePrefetch<K, S, D> pre;
    const int ix0 = (int)(ox0 * S - pad), hi = (int)Hi, wi = (int)Wi;
    pre.fetch(ip, (int)(ty0 * kTH * S - pad), ix0, hi, wi);
    float wr[K * K];
#pragma unroll
    for (int k = 0; k < K * K; ++k) wr[k] = w[c * K * K + (FLIP ? K * K - 1 - k : k)];
    const float b0 = BIAS ? bias[c] : 0.0f;
    const int t = threadIdx.x, r = t >> 3, c0 = (t & 7) * kPer;
    float mK = 0.0f, ms = 0.0f, mq = 0.0f;  // STATS: shift and shifted sums
    int mcnt = 0;
    HaloRows<K, D> halo;  // stride 1 only (k7 fwd 0.610 -> 0.603 ms, k3 d5 0.476 -> 0.442 ms)
    HaloFetch<K, D> hf;   // stride 1 only (k7 fwd 0.614 -> 0.556 ms, k3 0.413 -> 0.396 ms)
    if constexpr (S == 1) hf.init(ix0, wi);
    for (int64_t ty = ty0; ty < ty1; ++ty) {
        int lr0 = 0;
        if (ty > ty0) {
            __syncthreads();  // the previous tile's LDS reads are done
            if constexpr (S == 1) {
                halo.put(tile);
                lr0 = HaloRows<K, D>::O;
            }
        }
        pre.stash(tile, lr0);
        __syncthreads();
        if (ty + 1 < ty1) {
            if constexpr (S == 1) {
                const int y = (int)((ty + 1) * kTH - pad) + HaloRows<K, D>::O;
                hf.load(HaloFetch<K, D>::rsrc(ip, y, HaloFetch<K, D>::range(y, hi, wi), wi), pre.v);
                halo.take(tile);
            } else {
                pre.fetch(ip, (int)((ty + 1) * kTH * S - pad), ix0, hi, wi);
            }
        }
        float acc[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) acc[q] = b0;
#pragma unroll
        for (int ky = 0; ky < K; ++ky) {
            float seg[T::SL4];
            load_seg<K, S, D>(tile, r * S + ky * D, c0, seg);
#pragma unroll
            for (int kx = 0; kx < K; ++kx)
#pragma unroll
                for (int q = 0; q < kPer; ++q)
                    acc[q] = fmaf(wr[ky * K + kx], seg[q * S + kx * D], acc[q]);
        }
        const int64_t oy = ty * kTH + r;
        if (oy >= Ho) continue;
        float* orow = out + plane * Ho * Wo + oy * Wo;
        const int64_t ox = ox0 + c0;
        if constexpr (STATS) {
            const int nv = (int)min<int64_t>(kPer, Wo - ox);  // outputs stored (<= 0: none)
            if (ty == ty0 && nv > 0) mK = acc[0];
            if (nv == kPer) {  // a whole segment: the same sums without the tests
#pragma unroll
                for (int q = 0; q < kPer; ++q) {
                    const float d = acc[q] - mK;
                    ms += d;
                    mq = fmaf(d, d, mq);
                }
            } else {
#pragma unroll
                for (int q = 0; q < kPer; ++q)
                    if (q < nv) {
                        const float d = acc[q] - mK;
                        ms += d;
                        mq = fmaf(d, d, mq);
                    }
            }
            mcnt += max(nv, 0);
        }
        if (ox + kPer <= Wo && ((reinterpret_cast<uintptr_t>(orow + ox) & 15) == 0)) {
            f4* o4 = reinterpret_cast<f4*>(orow + ox);
            f4 v0 = {acc[0], acc[1], acc[2], acc[3]}, v1 = {acc[4], acc[5], acc[6], acc[7]};
            if (ACC) {
                v0 += o4[0];
                v1 += o4[1];
            }
            o4[0] = v0;
            o4[1] = v1;
        } else {
#pragma unroll
            for (int q = 0; q < kPer; ++q)
                if (ox + q < Wo) orow[ox + q] = ACC ? orow[ox + q] + acc[q] : acc[q];
        }
    }
    if constexpr (STATS) {
        const double2 m = block_moments<kDwThreads>(mK, ms, mq, mcnt, mom);
        if (t == 0) part[b] = m;
    }
}

template <int K, int S, int D, bool FLIP, bool ACC, bool BIAS, bool STATS = false>
__global__ __launch_bounds__(kDwThreads) void k_dw_conv(
    const float* __restrict__ in, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo,
    int64_t pad, int64_t tiles_x, int64_t tiles_y, int64_t tpp, int per,
    double2* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) float tile[Tile<K, S, D>::floats];
    __shared__ double mom[STATS ? 4 * kDwThreads / 64 : 1];
    dw_conv_body<K, S, D, FLIP, ACC, BIAS, STATS>(in, w, bias, out, C, Hi, Wi, Ho, Wo, pad,
                                                  tiles_x, tiles_y, tpp, per,
                                                  xcd_block(blockIdx.x, gridDim.x), tile, part,
                                                  mom);
}

// Stride 1, dilation 1, with RB consecutive output rows per thread (a
// 32*RB x 64 tile per step).  Input row i of a thread's window feeds its
// output row j through tap row ky = i - j, so each K+2-float row segment is
// read from LDS once for all RB rows: K + RB - 1 segment reads per RB x 8
// outputs instead of K * RB (at K = 7 and RB = 4, 10 instead of 28), for
// the same K*K FMAs per output.  Every output adds its terms in
// dw_conv_body's order (bias, then ky, then kx ascending), so the results
// are bit for bit the same.  STATS: dw_conv_body's statistics epilogue.
template <int K, bool FLIP, bool ACC, bool BIAS, int RB, bool STATS = false>
__device__ __forceinline__ void dw_conv_rb_body(
    const float* __restrict__ in, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo,
    int64_t pad, int64_t tiles_x, int64_t tiles_y, int64_t tpp, int per, int64_t b,
    float* __restrict__ tile, double2* __restrict__ part = nullptr, double* mom = nullptr) {
    using T = Tile<K, 1, 1, RB>;
    const int64_t plane = b / tpp, gix = b - plane * tpp;
    const int64_t c = plane % C;
    const int64_t tyg = gix / tiles_x, tx = gix - tyg * tiles_x;
    const int64_t ty0 = tyg * per, ty1 = min(ty0 + per, tiles_y);
    const int64_t ox0 = tx * kTW;
    const float* ip = in + plane * Hi * Wi;
    TilePrefetch<K, 1, 1, RB> pre;
    const int ix0 = (int)(ox0 - pad), hi = (int)Hi, wi = (int)Wi;
    pre.fetch(ip, (int)(ty0 * T::TH - pad), ix0, hi, wi);
    float wr[K * K];
#pragma unroll
    for (int k = 0; k < K * K; ++k) wr[k] = w[c * K * K + (FLIP ? K * K - 1 - k : k)];
    const float b0 = BIAS ? bias[c] : 0.0f;
    const int t = threadIdx.x, r0 = (t >> 3) * RB, c0 = (t & 7) * kPer;
    float mK = 0.0f, ms = 0.0f, mq = 0.0f;  // STATS: shift and shifted sums
    int mcnt = 0;
    HaloRows<K, 1, RB> halo;
    HaloFetch<K, 1, RB> hf;
    hf.init(ix0, wi);
    for (int64_t ty = ty0; ty < ty1; ++ty) {
        int lr0 = 0;
        if (ty > ty0) {
            __syncthreads();  // the previous tile's LDS reads are done
            halo.put(tile);
            lr0 = HaloRows<K, 1, RB>::O;
        }
        pre.stash(tile, lr0);
        __syncthreads();
        if (ty + 1 < ty1) {
            const int y = (int)((ty + 1) * T::TH - pad) + HaloRows<K, 1, RB>::O;
            hf.load(HaloFetch<K, 1, RB>::rsrc(ip, y, HaloFetch<K, 1, RB>::range(y, hi, wi), wi), pre.v);
            halo.take(tile);
        }
        float acc[RB][kPer];
#pragma unroll
        for (int j = 0; j < RB; ++j)
#pragma unroll
            for (int q = 0; q < kPer; ++q) acc[j][q] = b0;
#pragma unroll
        for (int i = 0; i < RB + K - 1; ++i) {
            float seg[T::SL4];
            load_seg<K, 1, 1, RB>(tile, r0 + i, c0, seg);
#pragma unroll
            for (int j = 0; j < RB; ++j) {
                const int ky = i - j;
                if (ky < 0 || ky >= K) continue;
#pragma unroll
                for (int kx = 0; kx < K; ++kx)
#pragma unroll
                    for (int q = 0; q < kPer; ++q)
                        acc[j][q] = fmaf(wr[ky * K + kx], seg[q + kx], acc[j][q]);
            }
        }
        const int64_t ox = ox0 + c0;
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int64_t oy = ty * T::TH + r0 + j;
            if (oy >= Ho) break;
            float* orow = out + plane * Ho * Wo + oy * Wo;
            if constexpr (STATS) {
                const int nv = (int)min<int64_t>(kPer, Wo - ox);  // outputs stored (<= 0: none)
                if (ty == ty0 && j == 0 && nv > 0) mK = acc[0][0];
                if (nv == kPer) {  // a whole segment: the same sums without the tests
#pragma unroll
                    for (int q = 0; q < kPer; ++q) {
                        const float d = acc[j][q] - mK;
                        ms += d;
                        mq = fmaf(d, d, mq);
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < kPer; ++q)
                        if (q < nv) {
                            const float d = acc[j][q] - mK;
                            ms += d;
                            mq = fmaf(d, d, mq);
                        }
                }
                mcnt += max(nv, 0);
            }
            if (ox + kPer <= Wo && ((reinterpret_cast<uintptr_t>(orow + ox) & 15) == 0)) {
                f4* o4 = reinterpret_cast<f4*>(orow + ox);
                f4 v0 = {acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
                f4 v1 = {acc[j][4], acc[j][5], acc[j][6], acc[j][7]};
                if (ACC) {
                    v0 += o4[0];
                    v1 += o4[1];
                }
                o4[0] = v0;
                o4[1] = v1;
            } else {
#pragma unroll
                for (int q = 0; q < kPer; ++q)
                    if (ox + q < Wo) orow[ox + q] = ACC ? orow[ox + q] + acc[j][q] : acc[j][q];
            }
        }
    }
    if constexpr (STATS) {
        const double2 m = block_moments<kDwThreads>(mK, ms, mq, mcnt, mom);
        if (t == 0) part[b] = m;
    }
}

template <int K, bool FLIP, bool ACC, bool BIAS, int RB, bool STATS = false>
__global__ __launch_bounds__(kDwThreads) void k_dw_conv_rb(
    const float* __restrict__ in, const float* __restrict__ w, const float* __restrict__ bias,
    float* __restrict__ out, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo,
    int64_t pad, int64_t tiles_x, int64_t tiles_y, int64_t tpp, int per,
    double2* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) float tile[Tile<K, 1, 1, RB>::floats];
    __shared__ double mom[STATS ? 4 * kDwThreads / 64 : 1];
    dw_conv_rb_body<K, FLIP, ACC, BIAS, RB, STATS>(in, w, bias, out, C, Hi, Wi, Ho, Wo, pad,
                                                   tiles_x, tiles_y, tpp, per,
                                                   xcd_block(blockIdx.x, gridDim.x), tile, part,
                                                   mom);
}

// Weight and bias gradient partials: a block walks `per` tiles down one
// plane (tile rows ty = tyg*per + i), accumulating in registers, then
// reduces once: part[g][c*(K*K+1) + k] with g = n*tpp + tyg*tiles_x + tx
// (tpp counting tile groups), k < K*K the tap sums sum dy*x, k = K*K the
// dy sum.  (The (K*K+1)-value block reduction costs about as much as a
// tile's FMAs for k7, so it is amortized over several tiles: 8 for K >= 7,
// 4 below, where more blocks per plane measured faster; fewer when that
// leaves the grid short of blocks, see wgrad_per.)

// With `direct` (one sample and one tile group per plane, so a block's sums
// are the whole sums) the block adds them into dw and db itself, exactly as
// k_dw_wgrad_finish would from its single partial, and no finish runs.
// (body of block b; `tile` holds Tile<K, S, D, 1, true>::floats floats)
template <int K, int S, int D>
__device__ __forceinline__ void dw_wgrad_body(
    const float* __restrict__ dy, const float* __restrict__ x, float* __restrict__ part,
    float* __restrict__ dw, float* __restrict__ db, bool direct, int64_t C, int64_t Hi,
    int64_t Wi, int64_t Ho, int64_t Wo, int64_t pad, int64_t tiles_x, int64_t tiles_y,
    int64_t tpp, int per, int64_t b, float* __restrict__ tile,
    float (*red)[K * K + 1]) {
    using T = Tile<K, S, D, 1, true>;
    constexpr int KK1 = K * K + 1;
    const int64_t plane = b / tpp, gix = b - plane * tpp;
    const int64_t n = plane / C, c = plane - n * C;
    const int64_t tyg = gix / tiles_x, tx = gix - tyg * tiles_x;
    const int t = threadIdx.x, r = t >> 3, c0 = (t & 7) * kPer;
    const float* xp = x + plane * Hi * Wi;
    const float* gp = dy + plane * Ho * Wo;
    float sw[KK1];
#pragma unroll
    for (int k = 0; k < KK1; ++k) sw[k] = 0.0f;
    // the next tile's x tile and dy values load while this tile's FMAs run
    const int64_t ty0 = tyg * per, ty1 = min(ty0 + per, tiles_y);
    const int64_t ox0 = tx * kTW;
    const int ix0 = (int)(ox0 * S - pad), hi = (int)Hi, wi = (int)Wi;
    TilePrefetch<K, S, D, 1, true> pre;
    float gn[kPer];
    // a thread's 8 dy values: two aligned 16-byte loads when the row is
    // inside the plane and 16-byte aligned, else element by element
    const bool dy_vec = Wo % 4 == 0 && (reinterpret_cast<uintptr_t>(gp) & 15) == 0;
    auto fetch_dy = [&](int64_t ty) {
        const int64_t oy = ty * kTH + r, ox = ox0 + c0;
        if (dy_vec && oy < Ho && ox + kPer <= Wo) {
            const f4* q = reinterpret_cast<const f4*>(gp + oy * Wo + ox);
            const f4 a = q[0], b = q[1];
            gn[0] = a.x, gn[1] = a.y, gn[2] = a.z, gn[3] = a.w;
            gn[4] = b.x, gn[5] = b.y, gn[6] = b.z, gn[7] = b.w;
            return;
        }
#pragma unroll
        for (int cc = 0; cc < kPer; ++cc)
            gn[cc] = (oy < Ho && ox + cc < Wo) ? gp[oy * Wo + ox + cc] : 0.0f;
    };
    pre.fetch(xp, (int)(ty0 * kTH * S - pad), ix0, hi, wi);
    fetch_dy(ty0);
    // shared halo rows for the dilated kernels only: at k3 d5 the weight
    // gradient went 0.432 -> 0.419 ms, while k3 d1 went 0.438 -> 0.451 and
    // k7 0.672 -> 0.677 ms (64 x 2048^2)
    constexpr bool kShare = S == 1 && D > 1;
    HaloRows<K, D, 1, true> halo;
    // whole later tiles through HaloFetch (stride 1 without shared rows,
    // K = 7: 0.558 -> 0.521 ms at 64 x 2048^2; k5 went 0.431 -> 0.448 ms
    // and at k3 the offsets cost two waves per SIMD, 64 -> 74 VGPRs)
    constexpr bool kWhole = S == 1 && !kShare && K >= 7;
    using WF = HaloFetch<K, D, 1, Tile<K, 1, D>::IH, true>;
    WF wf;
    if constexpr (kWhole) wf.init(ix0, wi);
    for (int64_t ty = ty0; ty < ty1; ++ty) {
        int lr0 = 0;
        if (ty > ty0) {
            __syncthreads();  // the previous tile's LDS reads are done
            if constexpr (kShare) {
                halo.put(tile);
                lr0 = HaloRows<K, D, 1, true>::O;
            }
        }
        pre.stash(tile, lr0);
        float g[kPer];
#pragma unroll
        for (int cc = 0; cc < kPer; ++cc) g[cc] = gn[cc];
        __syncthreads();
        if (ty + 1 < ty1) {
            if constexpr (kShare) {
                pre.fetch(xp, (int)((ty + 1) * kTH - pad), ix0, hi, wi, HaloRows<K, D, 1, true>::O);
                halo.take(tile);
            } else if constexpr (kWhole) {
                const int y = (int)((ty + 1) * kTH - pad);
                wf.load(WF::rsrc(xp, y, WF::range(y, hi, wi), wi), pre.v);
            } else {
                pre.fetch(xp, (int)((ty + 1) * kTH * S - pad), ix0, hi, wi);
            }
            fetch_dy(ty + 1);
        }
#pragma unroll
        for (int cc = 0; cc < kPer; ++cc) sw[K * K] += g[cc];
#pragma unroll
        for (int ky = 0; ky < K; ++ky) {
            float seg[T::SL4];
            load_seg<K, S, D, 1, true>(tile, r * S + ky * D, c0, seg);
#pragma unroll
            for (int kx = 0; kx < K; ++kx)
#pragma unroll
                for (int cc = 0; cc < kPer; ++cc)
                    sw[ky * K + kx] = fmaf(g[cc], seg[cc * S + kx * D], sw[ky * K + kx]);
        }
    }
    // block sum in a fixed order: wave trees, then the four waves in order
#pragma unroll
    for (int k = 0; k < KK1; ++k) {
        float v = sw[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off);
        sw[k] = v;
    }
    const int lane = t & 63, wv = t >> 6;
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < KK1; ++k) red[wv][k] = sw[k];
    }
    __syncthreads();
    if (t < KK1) {
        const float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
        if (direct) {
            float* o = t < K * K ? (dw ? dw + c * K * K + t : nullptr) : (db ? db + c : nullptr);
            if (o) *o = (float)((double)*o + (double)v);
        } else {
            part[(n * tpp + gix) * (C * KK1) + c * KK1 + t] = v;
        }
    }
}

template <int K, int S, int D>
__global__ __launch_bounds__(kDwThreads) void k_dw_wgrad(
    const float* __restrict__ dy, const float* __restrict__ x, float* __restrict__ part,
    float* __restrict__ dw, float* __restrict__ db, bool direct, int64_t C, int64_t Hi,
    int64_t Wi, int64_t Ho, int64_t Wo, int64_t pad, int64_t tiles_x, int64_t tiles_y,
    int64_t tpp, int per) {
    __shared__ __attribute__((aligned(16))) float tile[Tile<K, S, D, 1, true>::floats];
    __shared__ float red[kDwThreads / 64][K * K + 1];
    dw_wgrad_body<K, S, D>(dy, x, part, dw, db, direct, C, Hi, Wi, Ho, Wo, pad, tiles_x, tiles_y,
                           tpp, per, xcd_block(blockIdx.x, gridDim.x), tile, red);
}

// Input gradient for stride S > 1 over one 32 x 64 tile of dx per block:
//   dx[yi][xi] (+)= sum over taps with S | (yi + pad - ky*D) and
//   S | (xi + pad - kx*D) of w[ky][kx] * dy[(yi+pad-ky*D)/S][(xi+pad-kx*D)/S]
// (the reference's gather, k_conv2d_dw_backward_input).  The dy region the
// tile needs is staged in LDS (zeros outside dy, so no bounds tests in the
// sum).  For S = 2 the threads of a wave share one row parity and one
// column parity, so every tap test is uniform across the wave.
template <int K, int S, int D>
struct DTile {
    static constexpr int R = (kTH - 1 + (K - 1) * D) / S + 2;      // dy rows
    static constexpr int W = round4((kTW - 1 + (K - 1) * D) / S + 2);  // dy columns
};

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
    return a >= 0 ? a / b : -((-a + b - 1) / b);
}

// (body of block b; `tile` holds DTile R * W floats)
template <int K, int S, int D, bool ACC>
__device__ __forceinline__ void dw_dgrad_strided_body(
    const float* __restrict__ dy, const float* __restrict__ w, float* __restrict__ dx,
    int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo, int64_t pad, int64_t tiles_x,
    int64_t tiles_y, int64_t tpp, int per, int64_t b, float* __restrict__ tile) {
    using T = DTile<K, S, D>;
    constexpr int NR = (T::R * T::W + kDwThreads - 1) / kDwThreads;
    // `per` dx tiles down one plane per block (tiles over dx here); the dy
    // region of the next tile loads into registers while this one is summed
    const int64_t plane = b / tpp, gix = b - plane * tpp;
    const int64_t c = plane % C;
    const int64_t tyg = gix / tiles_x, tx = gix - tyg * tiles_x;
    const int64_t ty0 = tyg * per, ty1 = min(ty0 + per, tiles_y);
    const int64_t ox0 = tx * kTW;
    const int xlo = (int)floor_div(ox0 + pad - (K - 1) * D, S);
    const int ho = (int)Ho, wo = (int)Wo;
    const float* gp = dy + plane * Ho * Wo;
    float pv[NR];
    auto fetch = [&](int64_t ty) {
        const int ylo = (int)floor_div(ty * kTH + pad - (K - 1) * D, S);
        int t = (int)threadIdx.x;
        asm volatile("" : "+v"(t));  // recomputed per tile, not hoisted
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = t + k * kDwThreads;
            const int rr = i / T::W, cc = i - rr * T::W;
            const int yo = ylo + rr, xo = xlo + cc;
            float v = 0.0f;
            if (i < T::R * T::W && (unsigned)yo < (unsigned)ho && (unsigned)xo < (unsigned)wo)
                v = gp[yo * wo + xo];
            pv[k] = v;
        }
    };
    fetch(ty0);
    float wr[K * K];
#pragma unroll
    for (int k = 0; k < K * K; ++k) wr[k] = w[c * K * K + k];
    const int t = threadIdx.x, wv = t >> 6, l = t & 63;
    // rows 2*(l/8) + (wv & 1) + 16*(wv >> 1) give each wave one row parity
    const int r = S == 2 ? 2 * (l >> 3) + (wv & 1) + 16 * (wv >> 1) : t >> 3;
    const int c0 = (l & 7) * kPer;
    const int64_t xb = ox0 + c0;
    for (int64_t ty = ty0; ty < ty1; ++ty) {
        if (ty > ty0) __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = t + k * kDwThreads;
            if (i < T::R * T::W) tile[i] = pv[k];
        }
        __syncthreads();
        if (ty + 1 < ty1) fetch(ty + 1);
        const int64_t oy0 = ty * kTH;
        const int64_t ylo = floor_div(oy0 + pad - (K - 1) * D, S);
        const int64_t yi = oy0 + r;
        float acc[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int ky = 0; ky < K; ++ky) {
            const int64_t vy = yi + pad - ky * D;
            if (vy % S != 0) continue;
            const float* row = tile + (vy / S - ylo) * T::W;
#pragma unroll
            for (int kx = 0; kx < K; ++kx) {
                const float wk = wr[ky * K + kx];
#pragma unroll
                for (int q = 0; q < kPer; ++q) {
                    const int64_t vx = xb + q + pad - kx * D;
                    if (vx % S == 0) acc[q] = fmaf(wk, row[vx / S - xlo], acc[q]);
                }
            }
        }
        if (yi >= Hi) continue;
        float* orow = dx + plane * Hi * Wi + yi * Wi;
        if (xb + kPer <= Wi && ((reinterpret_cast<uintptr_t>(orow + xb) & 15) == 0)) {
            f4* o4 = reinterpret_cast<f4*>(orow + xb);
            f4 v0 = {acc[0], acc[1], acc[2], acc[3]}, v1 = {acc[4], acc[5], acc[6], acc[7]};
            if (ACC) {
                v0 += o4[0];
                v1 += o4[1];
            }
            o4[0] = v0;
            o4[1] = v1;
        } else {
#pragma unroll
            for (int q = 0; q < kPer; ++q)
                if (xb + q < Wi) orow[xb + q] = ACC ? orow[xb + q] + acc[q] : acc[q];
        }
    }
}

template <int K, int S, int D, bool ACC>
__global__ __launch_bounds__(kDwThreads) void k_dw_dgrad_strided(
    const float* __restrict__ dy, const float* __restrict__ w, float* __restrict__ dx,
    int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo, int64_t pad, int64_t tiles_x,
    int64_t tiles_y, int64_t tpp, int per) {
    __shared__ float tile[DTile<K, S, D>::R * DTile<K, S, D>::W];
    dw_dgrad_strided_body<K, S, D, ACC>(dy, w, dx, C, Hi, Wi, Ho, Wo, pad, tiles_x, tiles_y,
                                        tpp, per, xcd_block(blockIdx.x, gridDim.x), tile);
}

// The input gradient and the weight gradient of a small depthwise layer in
// one launch (each is a few microseconds of mostly fixed cost at such
// sizes): blocks [0, nbd) run the dx body (stride 1: the flipped-kernel
// convolution over dy; stride 2: the staged gather), the others the weight
// gradient's body on blocks b - nbd.  Each block does exactly what it does
// in its own kernel.  Used for small grids only: the union of the two
// bodies' registers would lower the larger grids' occupancy.
template <int K, int S, int D, bool ACC>
__global__ __launch_bounds__(kDwThreads) void k_dw_bwd_small(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ w,
    float* __restrict__ dx, float* __restrict__ part, float* __restrict__ dw,
    float* __restrict__ db, bool direct, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho,
    int64_t Wo, int64_t pad, int64_t dtx, int64_t dty, int64_t dtpp, int dper, int64_t wtx,
    int64_t wty, int64_t wtpp, int wper, int64_t nbd) {
    constexpr int TD = S == 1 ? Tile<K, 1, D>::floats : DTile<K, S, D>::R * DTile<K, S, D>::W;
    constexpr int TW = Tile<K, S, D, 1, true>::floats;  // dw_wgrad_body's tile
    __shared__ __attribute__((aligned(16))) float tile[TD > TW ? TD : TW];
    __shared__ float red[kDwThreads / 64][K * K + 1];
    const int64_t b = xcd_block(blockIdx.x, gridDim.x);
    if (b < nbd) {
        if constexpr (S == 1)
            dw_conv_body<K, 1, D, true, ACC, false>(dy, w, nullptr, dx, C, Ho, Wo, Hi, Wi,
                                                    (K - 1) * D - pad, dtx, dty, dtpp, dper, b,
                                                    tile);
        else
            dw_dgrad_strided_body<K, S, D, ACC>(dy, w, dx, C, Hi, Wi, Ho, Wo, pad, dtx, dty,
                                                dtpp, dper, b, tile);
    } else {
        dw_wgrad_body<K, S, D>(dy, x, part, dw, db, direct, C, Hi, Wi, Ho, Wo, pad, wtx, wty,
                               wtpp, wper, b - nbd, tile, red);
    }
}

// ======================================================================
// Fused backward of a depthwise CBA block whose convolution has stride 1
// and "same" padding, pad = (K-1)*D/2 (LKR.dw, the Ctx branches, Fuse's
// refine; blocks.cpp:449-500).  From the GroupNorm input z, the upstream
// gradient dy and the convolution input x, one kernel forms dz (the
// GroupNorm(+SiLU) input gradient, with k_bwd_dx's arithmetic from
// gn_math.hpp) over a tile and its halo in LDS and runs from it both
//   dx (+)= flip(w) (*) dz       the stride-1 adjoint (dw_conv_body's FMAs)
//   dw, db partials += dz (x) x  dw_wgrad_body's FMAs
// so dz never reaches HBM: z, dy and x are read once (with the halo) and
// dx written once, instead of GroupNorm dx (3T) + dgrad (2T) + wgrad (2T).
// dx or dw may be null (that product is skipped), not both.
// With "same" padding, the dz region a dx tile reads and the x region the
// weight gradient of that tile's dz reads are the same haloed tile (origin
// (oy0 - pad, ox0 - pad)), so one fetch serves the three tensors.  dz is
// zero outside the image (the adjoint's zero padding, and no weight-
// gradient term there).  A block walks `per` tiles down one plane, keeps
// the K*K+1 weight-gradient sums in registers across them and reduces once
// (dw_wgrad_body's partial layout, added by k_dw_wgrad_finish or, with
// `direct`, by the block itself).  The block of sample 0's first tile group
// of channel c also adds dgamma[c] / dbeta[c] from the GroupNorm plane
// sums in sample order (k_param_finish's sums).
// ======================================================================
// (The waves per SIMD the register budget allows without the folded
// finish, 5 at k3 and 4 at k5, held for the FOLD variants too: their extra
// scalar code would otherwise cost a wave.)
template <int K, int D, bool SILU, bool ACC, bool FOLD>
__global__ __launch_bounds__(kDwThreads, D == 1 ? (K == 3 ? 5 : K == 5 ? 4 : 1) : 1)
void k_dw_cba_bwd(
    const float* __restrict__ dy, const float* __restrict__ z, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ mean_lo,
    const double2* __restrict__ unit_sums, const double2* __restrict__ plane_sums,
    float* __restrict__ dgamma, float* __restrict__ dbeta, float* __restrict__ dx,
    float* __restrict__ part, float* __restrict__ dw, bool direct, int64_t N, int64_t C,
    int64_t G, int64_t H, int64_t W, int64_t tiles_x, int64_t tiles_y, int64_t tpp, int per,
    const double2* __restrict__ gn_part, int64_t gn_cpp) {
    using T = Tile<K, 1, D, 1, true>;
    constexpr int KK1 = K * K + 1;
    constexpr int PAD = (K - 1) * D / 2;
    constexpr int NR = (T::floats + kDwThreads - 1) / kDwThreads;
    static_assert(NR <= 32, "one mask bit per prefetched element");
    __shared__ __attribute__((aligned(16))) float tdz[T::floats];
    __shared__ __attribute__((aligned(16))) float tx[T::floats];
    __shared__ float red[kDwThreads / 64][KK1];
    __shared__ double2 fps[kFoldPlanes];  // the unit's plane sums (folded finish)
    __shared__ float fgam[kFoldPlanes];   // and their channels' gamma
    const int64_t blk = xcd_block(blockIdx.x, gridDim.x);
    const int64_t plane = blk / tpp, gix = blk - plane * tpp;
    const int64_t n = plane / C, c = plane - n * C;
    const int64_t tyg = gix / tiles_x, txg = gix - tyg * tiles_x;
    const int64_t ty0 = tyg * per, ty1 = min(ty0 + per, tiles_y);
    const int64_t ox0 = txg * kTW;
    const int64_t HW = H * W;
    const int hi = (int)H, wi = (int)W, ix0 = (int)ox0 - PAD;

    // this plane's GroupNorm dx coefficients, formed as k_bwd_dx forms them
    const int64_t cpg = C / G, u = n * G + c / cpg;
    const float mu = mean[u], r = rstd[u];
    const float e = mean_lo ? -mean_lo[u] * r : 0.0f;
    const float gm = gamma ? gamma[c] : 1.0f, bt = beta ? beta[c] : 0.0f;
    const float* zp = z + plane * HW;
    const float* gp = dy + plane * HW;
    const float* xp = x + plane * HW;
    // Consecutive tiles of the block share O = 2*PAD halo rows: local rows
    // [kTH, kTH + O) of one tile are rows [0, O) of the next.  Their dz and
    // x move to the top of the LDS tiles (through NS registers per thread)
    // instead of being fetched and formed again, so after the first tile a
    // block fetches and forms dz for its kTH new rows only.  The values are
    // the same either way.
    constexpr int O = 2 * PAD;
    constexpr int NS = (O * T::IWP + kDwThreads - 1) / kDwThreads;
    // this thread's elements (TilePrefetch's order) of local rows
    // [lr0, IH) of the haloed tile for the three tensors, and which of them
    // lie inside the image
    float pz[NR], pg[NR], px[NR];
    uint32_t inside = 0;
    auto fetch = [&](int64_t ty, int lr0) {
        const int iy0 = (int)(ty * kTH) - PAD;
        const int nel = (T::IH - lr0) * T::IWP, base = lr0 * T::IWP;
        int t = (int)threadIdx.x;
        asm volatile("" : "+v"(t));  // recomputed per tile, not hoisted
        inside = 0;
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = t + k * kDwThreads;
            const int li = base + i;
            const int rw = li / T::IWP, col = li - rw * T::IWP;
            const int yy = iy0 + rw, xx = ix0 + col;
            const bool in = i < nel && col < T::IW && (unsigned)yy < (unsigned)hi &&
                            (unsigned)xx < (unsigned)wi;
            float a = 0.0f, g = 0.0f, v = 0.0f;
            if (in) {
                const int off = yy * wi + xx;
                a = zp[off];
                g = gp[off];
                v = xp[off];
            }
            pz[k] = a;
            pg[k] = g;
            px[k] = v;
            inside |= (uint32_t)in << k;
        }
    };
    // the first tile's loads are in flight while the block folds the finish
    fetch(ty0, 0);
    // FOLD: the block folds the GroupNorm backward's finish from the
    // reduction's partials (unit_sums and plane_sums unused), with the
    // finish's own arithmetic.
    constexpr bool fold = FOLD;
    double2 S;
    if constexpr (fold) {
        bwd_plane_sums<kDwThreads>(gn_part, (int)(u * cpg), (int)cpg, (int)gn_cpp, fps, gamma,
                                   (int)C, fgam);
        __syncthreads();
        S = bwd_unit_sums(fps, fgam, (int)cpg, (int)gn_cpp);
    } else {
        S = unit_sums[u];
    }
    const double Md = (double)(cpg * HW);
    const float A = gm * r;
    const float B = (float)(-(double)r * S.x / Md);
    const float Dc = (float)(-(double)r * S.y / Md);
    if ((dgamma || dbeta) && n == 0 && gix == 0) {  // block-uniform
        double sa = 0.0, sb = 0.0;
        for (int64_t s = 0; s < N; ++s) {
            double2 v;
            if constexpr (fold) {
                __syncthreads();  // fps[0] read by every thread above
                bwd_plane_sums<kDwThreads>(gn_part, (int)(s * C + c), 1, (int)gn_cpp, fps);
                __syncthreads();
                v = fps[0];
            } else {
                v = plane_sums[s * C + c];
            }
            sa += v.x;
            sb += v.y;
        }
        if (threadIdx.x == 0) {
            if (dbeta) dbeta[c] = (float)((double)dbeta[c] + sa);
            if (dgamma) dgamma[c] = (float)((double)dgamma[c] + sb);
        }
    }

    float wr[K * K];
#pragma unroll
    for (int k = 0; k < K * K; ++k) wr[k] = w[c * K * K + K * K - 1 - k];  // flipped
    float sw[KK1];
#pragma unroll
    for (int k = 0; k < KK1; ++k) sw[k] = 0.0f;
    const int t = threadIdx.x, ro = t >> 3, c0 = (t & 7) * kPer;
    const bool want_dw = dw != nullptr;  // block-uniform; without it `part` is null
    const bool want_dx = dx != nullptr;

    float sdz[NS], sx[NS];  // the shared halo rows on their way to the top
    // The later tiles' new rows through HaloFetch for K >= 5 (at 64 x
    // 2048^2 k7 1.268 -> 1.185 ms, k5 0.928 -> 0.888 ms); at k3 its offsets
    // cost the kernel a wave per SIMD (96 -> 112 VGPRs; 0.842 -> 0.860 ms),
    // so k3 keeps fetch().
    constexpr bool kHF = K >= 5;
    HaloFetch<K, D, 1, kTH, true> hf;
    if constexpr (kHF) hf.init(ix0, wi);
    for (int64_t ty = ty0; ty < ty1; ++ty) {
        const int lr0 = ty > ty0 ? O : 0;
        if (ty > ty0) {
            __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int j = t + k * kDwThreads;
                if (j < O * T::IWP) {
                    tdz[j] = sdz[k];
                    tx[j] = sx[k];
                }
            }
        }
        const int nel = (T::IH - lr0) * T::IWP, base = lr0 * T::IWP;
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int i = t + k * kDwThreads;
            if (i < nel) {
                // every element computes and then selects (elements outside
                // the image are rare, so a branch only cost its exec-mask
                // code: k7 1.119 -> 1.103 ms at 64 x 2048^2)
                const float xh = fmaf(pz[k] - mu, r, e);
                const float dzs = SILU ? dsilu_fast(pg[k], fmaf(gm, xh, bt)) : pg[k];
                const float dv = fmaf(A, dzs, fmaf(Dc, xh, B));
                tdz[base + i] = (inside & (1u << k)) ? dv : 0.0f;
                tx[base + i] = px[k];
            }
        }
        __syncthreads();
        if (ty + 1 < ty1) {
            if constexpr (kHF) {
                const int y = (int)((ty + 1) * kTH) - PAD + O;
                const int lim = HaloFetch<K, D, 1, kTH, true>::range(y, hi, wi);
                hf.load(HaloFetch<K, D, 1, kTH, true>::rsrc(zp, y, lim, wi), pz);
                hf.load(HaloFetch<K, D, 1, kTH, true>::rsrc(gp, y, lim, wi), pg);
                hf.load(HaloFetch<K, D, 1, kTH, true>::rsrc(xp, y, lim, wi), px);
                inside = 0;
#pragma unroll
                for (int k = 0; k < HaloFetch<K, D, 1, kTH, true>::NF; ++k)
                    inside |= (uint32_t)(hf.off[k] < (uint32_t)lim) << k;
            } else {
                fetch(ty + 1, O);
            }
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const int j = t + k * kDwThreads;
                if (j < O * T::IWP) {
                    sdz[k] = tdz[kTH * T::IWP + j];
                    sx[k] = tx[kTH * T::IWP + j];
                }
            }
        }

        // dx for rows ty*32 + ro, columns ox0 + c0 .. +7
        float acc[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) acc[q] = 0.0f;
        if (want_dx) {
#pragma unroll
            for (int ky = 0; ky < K; ++ky) {
                float seg[T::SL4];
                load_seg<K, 1, D, 1, true>(tdz, ro + ky * D, c0, seg);
#pragma unroll
                for (int kx = 0; kx < K; ++kx)
#pragma unroll
                    for (int q = 0; q < kPer; ++q)
                        acc[q] = fmaf(wr[ky * K + kx], seg[q + kx * D], acc[q]);
            }
        }
        // weight gradient: this tile's dz (the halo's interior) against x
        if (want_dw) {
            float g[kPer];
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                g[q] = tdz[(ro + PAD) * T::IWP + c0 + q + PAD];
                sw[K * K] += g[q];
            }
#pragma unroll
            for (int ky = 0; ky < K; ++ky) {
                float seg[T::SL4];
                load_seg<K, 1, D, 1, true>(tx, ro + ky * D, c0, seg);
#pragma unroll
                for (int kx = 0; kx < K; ++kx)
#pragma unroll
                    for (int q = 0; q < kPer; ++q)
                        sw[ky * K + kx] = fmaf(g[q], seg[q + kx * D], sw[ky * K + kx]);
            }
        }
        const int64_t oy = ty * kTH + ro;
        if (!want_dx || oy >= H) continue;
        float* orow = dx + plane * HW + oy * W;
        const int64_t ox = ox0 + c0;
        if (ox + kPer <= W && ((reinterpret_cast<uintptr_t>(orow + ox) & 15) == 0)) {
            f4* o4 = reinterpret_cast<f4*>(orow + ox);
            f4 v0 = {acc[0], acc[1], acc[2], acc[3]}, v1 = {acc[4], acc[5], acc[6], acc[7]};
            if (ACC) {
                v0 += o4[0];
                v1 += o4[1];
            }
            o4[0] = v0;
            o4[1] = v1;
        } else {
#pragma unroll
            for (int q = 0; q < kPer; ++q)
                if (ox + q < W) orow[ox + q] = ACC ? orow[ox + q] + acc[q] : acc[q];
        }
    }
    if (!want_dw) return;
    // block sum of the weight-gradient terms in a fixed order (dw_wgrad_body's)
#pragma unroll
    for (int k = 0; k < KK1; ++k) {
        float v = sw[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off);
        sw[k] = v;
    }
    const int lane = t & 63, wv = t >> 6;
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < KK1; ++k) red[wv][k] = sw[k];
    }
    __syncthreads();
    if (t < KK1) {
        const float v = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
        if (direct) {
            if (t < K * K) dw[c * K * K + t] = (float)((double)dw[c * K * K + t] + (double)v);
        } else {
            part[(n * tpp + gix) * (C * KK1) + c * KK1 + t] = v;
        }
    }
}

// ---- generic kernels (any K, S, D): one thread per output element --------

template <bool FLIP, bool ACC>
__global__ void k_dw_conv_generic(const float* __restrict__ in, const float* __restrict__ w,
                                  const float* __restrict__ bias, float* __restrict__ out,
                                  int64_t NC, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho,
                                  int64_t Wo, int64_t K, int64_t pad, int64_t S, int64_t D) {
    const int64_t total = NC * Ho * Wo;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t xo = i % Wo, tt = i / Wo, yo = tt % Ho, plane = tt / Ho, c = plane % C;
        const float* ip = in + plane * Hi * Wi;
        const float* wc = w + c * K * K;
        float acc = bias ? bias[c] : 0.0f;
        for (int64_t ky = 0; ky < K; ++ky) {
            const int64_t yi = yo * S - pad + ky * D;
            if (yi < 0 || yi >= Hi) continue;
            for (int64_t kx = 0; kx < K; ++kx) {
                const int64_t xi = xo * S - pad + kx * D;
                if (xi < 0 || xi >= Wi) continue;
                const int64_t k = ky * K + kx;
                acc = fmaf(wc[FLIP ? K * K - 1 - k : k], ip[yi * Wi + xi], acc);
            }
        }
        out[i] = ACC ? out[i] + acc : acc;
    }
}

// dx (+)= gather of dy over the taps of each input element (any stride).
template <bool ACC>
__global__ void k_dw_dx_gather(const float* __restrict__ dy, const float* __restrict__ w,
                               float* __restrict__ dx, int64_t NC, int64_t C, int64_t Hi,
                               int64_t Wi, int64_t Ho, int64_t Wo, int64_t K, int64_t pad,
                               int64_t S, int64_t D) {
    const int64_t total = NC * Hi * Wi;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t xi = i % Wi, tt = i / Wi, yi = tt % Hi, plane = tt / Hi, c = plane % C;
        const float* gp = dy + plane * Ho * Wo;
        const float* wc = w + c * K * K;
        float acc = 0.0f;
        for (int64_t ky = 0; ky < K; ++ky) {
            const int64_t nh = yi + pad - ky * D;
            if (nh < 0 || nh % S) continue;
            const int64_t yo = nh / S;
            if (yo >= Ho) continue;
            for (int64_t kx = 0; kx < K; ++kx) {
                const int64_t nw = xi + pad - kx * D;
                if (nw < 0 || nw % S) continue;
                const int64_t xo = nw / S;
                if (xo < Wo) acc = fmaf(gp[yo * Wo + xo], wc[ky * K + kx], acc);
            }
        }
        dx[i] = ACC ? dx[i] + acc : acc;
    }
}

// One block per (c, k): k < K*K the tap sum of dy*x over all samples and
// outputs, k = K*K the dy sum; added into dw / db (fixed order).
__global__ __launch_bounds__(256) void k_dw_wgrad_generic(
    const float* __restrict__ dy, const float* __restrict__ x, float* __restrict__ dw,
    float* __restrict__ db, int64_t N, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho, int64_t Wo,
    int64_t K, int64_t pad, int64_t S, int64_t D) {
    __shared__ double red[256];
    const int64_t KK1 = K * K + 1;
    const int64_t c = blockIdx.x / KK1, k = blockIdx.x - c * KK1;
    if ((k < K * K && !dw) || (k == K * K && !db)) return;
    const int64_t ky = k / K, kx = k - ky * K;
    double acc = 0.0;
    for (int64_t n = 0; n < N; ++n) {
        const float* gp = dy + (n * C + c) * Ho * Wo;
        const float* xp = x + (n * C + c) * Hi * Wi;
        for (int64_t i = threadIdx.x; i < Ho * Wo; i += 256) {
            if (k == K * K) {
                acc += (double)gp[i];
                continue;
            }
            const int64_t yo = i / Wo, xo = i - yo * Wo;
            const int64_t yi = yo * S - pad + ky * D, xi = xo * S - pad + kx * D;
            if (yi >= 0 && yi < Hi && xi >= 0 && xi < Wi)
                acc += (double)gp[i] * (double)xp[yi * Wi + xi];
        }
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        float* o = k < K * K ? &dw[c * K * K + k] : &db[c];
        *o = (float)((double)*o + red[0]);
    }
}

// dw[c*K*K + k] += sum_g part[g][c*KK1 + k], db[c] += sum_g part[g][c*KK1 + K*K]
// (float64, g ascending in 16 fixed segments; see k_sum_partials).
__global__ __launch_bounds__(1024) void k_dw_wgrad_finish(const float* __restrict__ part,
                                                          float* __restrict__ dw,
                                                          float* __restrict__ db, int64_t E,
                                                          int64_t G, int64_t KK1) {
    __shared__ double lds[16][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const int64_t g0 = wv * G / 16, g1 = (wv + 1) * G / 16;
    const double sum = e < E ? segment_sum(part, E, e, g0, g1) : 0.0;
    lds[wv][lane] = sum;
    __syncthreads();
    if (wv == 0 && e < E) {
        double tsum = 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) tsum += lds[i][lane];
        const int64_t c = e / KK1, k = e - c * KK1;
        float* o = k < KK1 - 1 ? (dw ? &dw[c * (KK1 - 1) + k] : nullptr) : db ? &db[c] : nullptr;
        if (o) *o = (float)((double)*o + tsum);
    }
}

template <typename F>
void bsel(bool b, F&& f) {
    if (b)
        f(std::true_type{});
    else
        f(std::false_type{});
}

template <int K, int S, int D>
struct Cfg {
    static constexpr int k = K, s = S, d = D;
};

// Calls f(Cfg<K,S,D>{}) for a configuration with a fast kernel; false if
// there is none.
template <typename F>
bool fast_cfg(int64_t K, int64_t S, int64_t D, F&& f) {
    if (K == 3 && S == 1 && D == 1) return f(Cfg<3, 1, 1>{}), true;
    if (K == 3 && S == 2 && D == 1) return f(Cfg<3, 2, 1>{}), true;
    if (K == 5 && S == 1 && D == 1) return f(Cfg<5, 1, 1>{}), true;
    if (K == 7 && S == 1 && D == 1) return f(Cfg<7, 1, 1>{}), true;
    if (K == 3 && S == 1 && D == 2) return f(Cfg<3, 1, 2>{}), true;
    if (K == 3 && S == 1 && D == 3) return f(Cfg<3, 1, 3>{}), true;
    if (K == 3 && S == 1 && D == 5) return f(Cfg<3, 1, 5>{}), true;
    return false;
}

// Output rows per thread of the stride-1, dilation-1 forward / input
// gradient: 2 for K = 3 and 5 (k_dw_conv_rb), 1 for K = 7 and elsewhere
// (k_dw_conv).  At 64 x 2048^2, fwd / dgrad for 1 / 2 / 3 / 4 rows: k3
// 0.432 / 0.414 / 0.465 / 0.432 and 0.449 / 0.425 / 0.477 / 0.443 ms, k5
// 0.452 / 0.449 / 0.500 / 0.468 and 0.459 / 0.447 / 0.505 / 0.472 ms, k7
// 0.605 / 0.612 / - / 0.653 ms (its FMAs, not its LDS reads, bound it, and
// 4 rows take 215 VGPRs: 2 waves per SIMD).  Three rows leave a ragged
// 96-row tile at the bottom of every power-of-two plane.
template <int K>
constexpr int conv_rb() {
    return K == 3 || K == 5 ? 2 : 1;
}

int conv_rows_per_thread(int64_t K, int64_t S, int64_t D) {
    if (S != 1 || D != 1) return 1;
    if (K == 3) return conv_rb<3>();
    if (K == 5) return conv_rb<5>();
    if (K == 7) return conv_rb<7>();
    return 1;
}

int64_t tiles_of(int64_t H, int64_t W, int64_t* tiles_x) {
    *tiles_x = (W + kTW - 1) / kTW;
    return ((H + kTH - 1) / kTH) * *tiles_x;
}

// k_dw_conv addresses a plane with 32-bit element offsets, and HaloFetch
// the rows of a tile with 31-bit byte offsets (64 rows: 2^23 columns).
bool planes_fit_32(const DwShape& sh) {
    const int64_t lim = (int64_t)1 << 31;
    return sh.Hi * sh.Wi < lim && sh.Ho * sh.Wo < lim && sh.Hi < lim &&
           sh.Wi < ((int64_t)1 << 23) && sh.Wo < ((int64_t)1 << 23);
}

// Tile rows per block of k_dw_conv over `planes` planes of H x W outputs
// (the next tile's input loads overlap the current tile's FMAs, and a block
// loads its K*K weights, fetches its first tile whole and combines its
// statistics once): 16 at K = 7, 8 at K = 5, 4 below, halved while the grid
// would hold fewer than 4096 blocks.  At 64 x 2048^2 (one box, two rounds),
// 4 / 8 / 16 tiles: k7 forward 0.543 / 0.512 / 0.506 ms, with statistics
// 0.588 / 0.536 / 0.517 ms, input gradient 0.546 / 0.515 / 0.508 ms; k5
// forward 0.419 / 0.412 / 0.426 ms; k3 0.392 / 0.409 / 0.426 ms.  Returns
// the tile groups per plane; *per the rows per group.
int conv_per(int64_t K) { return K >= 7 ? 16 : K == 5 ? 8 : 4; }

int64_t conv_groups(int64_t planes, int64_t H, int64_t W, int64_t* tiles_x, int64_t* tiles_y,
                    int* per, int64_t K, int64_t th = kTH) {
    *tiles_x = (W + kTW - 1) / kTW;
    *tiles_y = (H + th - 1) / th;
    int p = conv_per(K);
    while (p > 1 && planes * ((*tiles_y + p - 1) / p) * *tiles_x < 4096) p /= 2;
    *per = p;
    return ((*tiles_y + p - 1) / p) * *tiles_x;
}

// Layers whose dx and weight-gradient grids hold at most this many blocks
// together run both in one launch (k_dw_bwd_small).
constexpr int64_t kDwFuseBlocks = 2048;

unsigned grid_stride_blocks(int64_t total) {
    const int64_t b = (total + 255) / 256;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, 65536));
}

}  // namespace

bool dw_has_fast(int64_t K, int64_t S, int64_t D) {
    return fast_cfg(K, S, D, [](auto) {});
}

// Tiles per weight-gradient block: 64 for K >= 7, 16 for K = 5, 4 below
// (each block reduces its K*K+1 sums once, which at k7 costs as much as a
// few tiles' FMAs), halved while the grid would hold fewer than 2048 blocks
// (a block walks its tiles one after another: few large planes, e.g. 16
// channels at 256 x 256 with k3 s2, ran 64 blocks of 4 tiles in 55 us).
// At 64 x 2048^2, k7 8 / 16 / 32 tiles: 0.704 / 0.628 / 0.585 ms, and with
// the XCD runs of 32 tiles 16 / 32 / 64: 0.521 / 0.487 / 0.478 ms; k5 4 / 8
// / 16: 0.524 / 0.463 / 0.448 ms (0.446 -> 0.432 ms for 8 -> 16 on another
// box).  K >= 5 matches the fused CBA backward's grouping, so both add the
// same partial sums in the same order.
int64_t wgrad_per(const DwShape& sh) {
    int64_t per = sh.K >= 7 ? 64 : sh.K >= 5 ? 16 : 4;
    const int64_t tx = (sh.Wo + kTW - 1) / kTW, ty = (sh.Ho + kTH - 1) / kTH;
    while (per > 1 && sh.N * sh.C * ((ty + per - 1) / per) * tx < 2048) per /= 2;
    return per;
}

// Tile groups of the weight-gradient kernel over an Ho x Wo plane.
int64_t wgrad_groups(const DwShape& sh, int64_t per, int64_t* tiles_x, int64_t* tiles_y) {
    *tiles_x = (sh.Wo + kTW - 1) / kTW;
    *tiles_y = (sh.Ho + kTH - 1) / kTH;
    return ((*tiles_y + per - 1) / per) * *tiles_x;
}

size_t dw_bwd_workspace_bytes(const DwShape& sh) {
    if (!dw_has_fast(sh.K, sh.S, sh.D)) return 0;
    int64_t tx = 0, ty = 0;
    const int64_t tpp = wgrad_groups(sh, wgrad_per(sh), &tx, &ty);
    const size_t b = sizeof(float) * (size_t)(sh.N * tpp) * (size_t)(sh.C * (sh.K * sh.K + 1));
    return (b + 255) & ~(size_t)255;
}

int64_t dw_grid_blocks(const DwShape& sh, bool output_tiles) {
    int64_t tx = 0;
    const int64_t tpp = output_tiles ? tiles_of(sh.Ho, sh.Wo, &tx) : tiles_of(sh.Hi, sh.Wi, &tx);
    return sh.N * sh.C * tpp;
}

bool dw_stats_geometry(const DwShape& sh, DwStatsGeom* g) {
    if (!planes_fit_32(sh) || !dw_has_fast(sh.K, sh.S, sh.D)) return false;
    int64_t tiles_y = 0;
    int per = 1;
    const int rb = conv_rows_per_thread(sh.K, sh.S, sh.D);
    g->tpp = conv_groups(sh.N * sh.C, sh.Ho, sh.Wo, &g->tiles_x, &tiles_y, &per, sh.K,
                         (int64_t)kTH * rb);
    g->rows = (int64_t)per * kTH * rb;
    return true;
}

hipError_t launch_dw_forward(const DwShape& sh, const float* x, const float* w,
                             const float* bias, float* y, hipStream_t s, double2* part) {
    if (sh.N * sh.C * sh.Ho * sh.Wo == 0) return hipSuccess;
    DwStatsGeom geom;
    if (part && !dw_stats_geometry(sh, &geom)) return hipErrorInvalidValue;  // no tiled kernel
    int64_t tiles_x = 0, tiles_y = 0;
    int per = 1;
    const int rb = conv_rows_per_thread(sh.K, sh.S, sh.D);
    const int64_t tpp =
        conv_groups(sh.N * sh.C, sh.Ho, sh.Wo, &tiles_x, &tiles_y, &per, sh.K, (int64_t)kTH * rb);
    const int tok = prof_begin(s, part ? "dw_conv_stats" : "dw_conv");
    const bool fast = planes_fit_32(sh) && fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
        using CF = decltype(cf);
        bsel(bias != nullptr, [&](auto B) {
            bsel(part != nullptr, [&](auto ST) {
                const dim3 grid((unsigned)(sh.N * sh.C * tpp));
                if constexpr (CF::s == 1 && CF::d == 1 && conv_rb<CF::k>() > 1) {
                    k_dw_conv_rb<CF::k, false, false, B(), conv_rb<CF::k>(), ST()>
                        <<<grid, kDwThreads, 0, s>>>(x, w, bias, y, sh.C, sh.Hi, sh.Wi, sh.Ho,
                                                     sh.Wo, sh.pad, tiles_x, tiles_y, tpp, per,
                                                     part);
                } else {
                    k_dw_conv<CF::k, CF::s, CF::d, false, false, B(), ST()>
                        <<<grid, kDwThreads, 0, s>>>(x, w, bias, y, sh.C, sh.Hi, sh.Wi, sh.Ho,
                                                     sh.Wo, sh.pad, tiles_x, tiles_y, tpp, per,
                                                     part);
                }
            });
        });
    });
    if (!fast)
        k_dw_conv_generic<false, false>
            <<<grid_stride_blocks(sh.N * sh.C * sh.Ho * sh.Wo), 256, 0, s>>>(
                x, w, bias, y, sh.N * sh.C, sh.C, sh.Hi, sh.Wi, sh.Ho, sh.Wo, sh.K, sh.pad, sh.S,
                sh.D);
    prof_end(s, tok);
    return hipGetLastError();
}

hipError_t launch_dw_backward(const DwShape& sh, const float* dy, const float* x,
                              const float* w, float* dx, float* dw, float* db,
                              bool accumulate_dx, void* ws, hipStream_t s) {
    if (sh.N * sh.C == 0) return hipSuccess;
    if (dx && (dw || db) && sh.Hi * sh.Wi > 0 && sh.Ho * sh.Wo > 0 && planes_fit_32(sh)) {
        // a small layer: dx and the weight gradient in one launch
        int64_t dtx = 0, dty = 0, wtx = 0, wty = 0;
        int dper = 1;
        const int64_t dtpp = conv_groups(sh.N * sh.C, sh.Hi, sh.Wi, &dtx, &dty, &dper, sh.K);
        const int64_t wper = wgrad_per(sh);
        const int64_t wtpp = wgrad_groups(sh, wper, &wtx, &wty);
        const int64_t nbd = sh.N * sh.C * dtpp, nbw = sh.N * sh.C * wtpp;
        const bool direct = sh.N * wtpp == 1;
        float* part = static_cast<float*>(ws);
        bool fused = false;
        if (nbd + nbw <= kDwFuseBlocks && (sh.S == 1 || sh.S == 2)) {
            const int tok = prof_begin(s, "dw_conv_bwd_small");
            fused = fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
                using CF = decltype(cf);
                bsel(accumulate_dx, [&](auto A) {
                    k_dw_bwd_small<CF::k, CF::s, CF::d, A()>
                        <<<dim3((unsigned)(nbd + nbw)), kDwThreads, 0, s>>>(
                            dy, x, w, dx, part, dw, db, direct, sh.C, sh.Hi, sh.Wi, sh.Ho, sh.Wo,
                            sh.pad, dtx, dty, dtpp, dper, wtx, wty, wtpp, (int)wper, nbd);
                });
            });
            prof_end(s, tok);
        }
        if (fused) {
            if (!direct) {
                const int64_t KK1 = sh.K * sh.K + 1, E = sh.C * KK1;
                hipError_t qe = hipSuccess;
                if (weight_finish_queue({part, dw, db, E, sh.N * wtpp, KK1}, s, &qe))
                    return qe != hipSuccess ? qe : hipGetLastError();
                const int tok = prof_begin(s, "dw_conv_wgrad_finish");
                k_dw_wgrad_finish<<<dim3((unsigned)((E + 63) / 64)), 1024, 0, s>>>(
                    part, dw, db, E, sh.N * wtpp, KK1);
                prof_end(s, tok);
            }
            return hipGetLastError();
        }
    }
    if (dx && sh.Hi * sh.Wi > 0) {
        const int tok = prof_begin(s, "dw_conv_dgrad");
        bool done = false;
        if (sh.S == 1) {
            // the adjoint of a stride-1 convolution: the flipped kernel over
            // dy with pad' = (K-1)*D - pad, producing dx's plane
            int64_t tiles_x = 0, tiles_y = 0;
            int per = 1;
            const int rb = conv_rows_per_thread(sh.K, sh.S, sh.D);
            const int64_t tpp = conv_groups(sh.N * sh.C, sh.Hi, sh.Wi, &tiles_x, &tiles_y, &per, sh.K,
                                            (int64_t)kTH * rb);
            const int64_t padf = (sh.K - 1) * sh.D - sh.pad;
            done = planes_fit_32(sh) && fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
                using CF = decltype(cf);
                bsel(accumulate_dx, [&](auto A) {
                    const dim3 grid((unsigned)(sh.N * sh.C * tpp));
                    if constexpr (CF::s == 1 && CF::d == 1 && conv_rb<CF::k>() > 1) {
                        k_dw_conv_rb<CF::k, true, A(), false, conv_rb<CF::k>()>
                            <<<grid, kDwThreads, 0, s>>>(dy, w, nullptr, dx, sh.C, sh.Ho, sh.Wo,
                                                         sh.Hi, sh.Wi, padf, tiles_x, tiles_y,
                                                         tpp, per, nullptr);
                    } else {
                        k_dw_conv<CF::k, CF::s, CF::d, true, A(), false>
                            <<<grid, kDwThreads, 0, s>>>(dy, w, nullptr, dx, sh.C, sh.Ho, sh.Wo,
                                                         sh.Hi, sh.Wi, padf, tiles_x, tiles_y,
                                                         tpp, per, nullptr);
                    }
                });
            });
        }
        if (!done && sh.S > 1) {
            int64_t tiles_x = 0, tiles_y = 0;
            int per = 1;
            const int64_t tpp = conv_groups(sh.N * sh.C, sh.Hi, sh.Wi, &tiles_x, &tiles_y, &per, sh.K);
            done = planes_fit_32(sh) && fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
                using CF = decltype(cf);
                if constexpr (CF::s > 1) {
                    bsel(accumulate_dx, [&](auto A) {
                        k_dw_dgrad_strided<CF::k, CF::s, CF::d, A()>
                            <<<dim3((unsigned)(sh.N * sh.C * tpp)), kDwThreads, 0, s>>>(
                                dy, w, dx, sh.C, sh.Hi, sh.Wi, sh.Ho, sh.Wo, sh.pad, tiles_x,
                                tiles_y, tpp, per);
                    });
                }
            });
        }
        if (!done) {
            bsel(accumulate_dx, [&](auto A) {
                k_dw_dx_gather<A()><<<grid_stride_blocks(sh.N * sh.C * sh.Hi * sh.Wi), 256, 0,
                                      s>>>(dy, w, dx, sh.N * sh.C, sh.C, sh.Hi, sh.Wi, sh.Ho,
                                           sh.Wo, sh.K, sh.pad, sh.S, sh.D);
            });
        }
        prof_end(s, tok);
    }
    if ((dw || db) && sh.Ho * sh.Wo > 0) {
        const int64_t KK1 = sh.K * sh.K + 1;
        int64_t tiles_x = 0, tiles_y = 0;
        const int64_t per = wgrad_per(sh);
        const int64_t tpp = wgrad_groups(sh, per, &tiles_x, &tiles_y);
        float* part = static_cast<float*>(ws);
        const bool direct = sh.N * tpp == 1;
        int tok = prof_begin(s, "dw_conv_wgrad");
        const bool fast = planes_fit_32(sh) && fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
            using CF = decltype(cf);
            k_dw_wgrad<CF::k, CF::s, CF::d>
                <<<dim3((unsigned)(sh.N * sh.C * tpp)), kDwThreads, 0, s>>>(
                    dy, x, part, dw, db, direct, sh.C, sh.Hi, sh.Wi, sh.Ho, sh.Wo, sh.pad,
                    tiles_x, tiles_y, tpp, (int)per);
        });
        prof_end(s, tok);
        if (fast && direct) return hipGetLastError();  // the blocks added the sums
        if (fast) {
            hipError_t qe = hipSuccess;
            if (weight_finish_queue({part, dw, db, sh.C * KK1, sh.N * tpp, KK1}, s, &qe))
                return qe != hipSuccess ? qe : hipGetLastError();
        }
        tok = prof_begin(s, "dw_conv_wgrad_finish");
        if (fast) {
            const int64_t E = sh.C * KK1;
            k_dw_wgrad_finish<<<dim3((unsigned)((E + 63) / 64)), 1024, 0, s>>>(
                part, dw, db, E, sh.N * tpp, KK1);
        } else {
            k_dw_wgrad_generic<<<dim3((unsigned)(sh.C * KK1)), 256, 0, s>>>(
                dy, x, dw, db, sh.N, sh.C, sh.Hi, sh.Wi, sh.Ho, sh.Wo, sh.K, sh.pad, sh.S, sh.D);
        }
        prof_end(s, tok);
    }
    return hipGetLastError();
}

bool dw_cba_fused_fits(const DwShape& sh) {
    return sh.S == 1 && sh.Ho == sh.Hi && sh.Wo == sh.Wi && (sh.K - 1) * sh.D % 2 == 0 &&
           sh.pad == (sh.K - 1) * sh.D / 2 && sh.Hi * sh.Wi > 0 && planes_fit_32(sh) &&
           dw_has_fast(sh.K, sh.S, sh.D);
}

namespace {
// Tiles per block of the fused CBA backward: 64 for K >= 7 and 16 for K = 5
// (the block reduces its K*K+1 weight-gradient sums once per block; the
// stand-alone weight gradient groups the same tiles), 2 for K = 3 (more
// blocks), halved while the grid would hold fewer than 2048 blocks.  At
// 64 x 2048^2, k7 8 / 16 / 32 tiles: 1.39 / 1.31 / 1.29 ms (later kernels,
// with the XCD runs of 32 tiles, 16 / 32 / 64: 1.144 / 1.107 / 1.103 ms); k5
// 16 / 8 / 4 / 2: 0.934 / 0.934 / 1.04 / 1.14 ms; k3 4 / 2: 0.88 / 0.85 ms.
int64_t dw_cba_per(const DwShape& sh, int64_t* tiles_x, int64_t* tiles_y, int64_t* tpp) {
    *tiles_x = (sh.Wi + kTW - 1) / kTW;
    *tiles_y = (sh.Hi + kTH - 1) / kTH;
    int64_t per = sh.K >= 7 ? 64 : sh.K >= 5 ? 16 : 2;
    while (per > 1 && sh.N * sh.C * ((*tiles_y + per - 1) / per) * *tiles_x < 2048) per /= 2;
    *tpp = ((*tiles_y + per - 1) / per) * *tiles_x;
    return per;
}
}  // namespace

size_t dw_cba_part_bytes(const DwShape& sh) {
    int64_t tx = 0, ty = 0, tpp = 0;
    dw_cba_per(sh, &tx, &ty, &tpp);
    const size_t b = sizeof(float) * (size_t)(sh.N * tpp) * (size_t)(sh.C * (sh.K * sh.K + 1));
    return (b + 255) & ~(size_t)255;
}

int64_t dw_cba_grid_blocks(const DwShape& sh) {
    int64_t tx = 0, ty = 0, tpp = 0;
    dw_cba_per(sh, &tx, &ty, &tpp);
    return sh.N * sh.C * tpp;
}

hipError_t launch_dw_cba_backward(const DwShape& sh, const DwCbaArgs& a, int64_t G, bool silu,
                                  bool accumulate_dx, hipStream_t s) {
    if (sh.N * sh.C * sh.Hi * sh.Wi == 0) return hipSuccess;
    int64_t tiles_x = 0, tiles_y = 0, tpp = 0;
    const int64_t per = dw_cba_per(sh, &tiles_x, &tiles_y, &tpp);
    const bool direct = sh.N * tpp == 1;
    float* part = a.dw ? a.part : nullptr;
    int tok = prof_begin(s, "dw_cba_bwd");
    fast_cfg(sh.K, sh.S, sh.D, [&](auto cf) {
        using CF = decltype(cf);
        if constexpr (CF::s == 1) {
            bsel(silu, [&](auto SI) {
                bsel(accumulate_dx, [&](auto AC) { bsel(a.unit_sums == nullptr, [&](auto FO) {
                    k_dw_cba_bwd<CF::k, CF::d, SI(), AC(), FO()>
                        <<<dim3((unsigned)(sh.N * sh.C * tpp)), kDwThreads, 0, s>>>(
                            a.dy, a.z, a.x, a.w, a.gamma, a.beta, a.mean, a.rstd, a.mean_lo,
                            a.unit_sums, a.plane_sums, a.dgamma, a.dbeta, a.dx, part, a.dw,
                            direct, sh.N, sh.C, G, sh.Hi, sh.Wi, tiles_x, tiles_y, tpp,
                            (int)per, a.gn_part, a.gn_cpp);
                }); });
            });
        }
    });
    prof_end(s, tok);
    if (a.dw && !direct) {
        const int64_t KK1 = sh.K * sh.K + 1, E = sh.C * KK1;
        hipError_t qe = hipSuccess;
        if (weight_finish_queue({part, a.dw, nullptr, E, sh.N * tpp, KK1}, s, &qe))
            return qe != hipSuccess ? qe : hipGetLastError();
        tok = prof_begin(s, "dw_cba_wgrad_finish");
        k_dw_wgrad_finish<<<dim3((unsigned)((E + 63) / 64)), 1024, 0, s>>>(part, a.dw, nullptr, E,
                                                                           sh.N * tpp, KK1);
        prof_end(s, tok);
    }
    return hipGetLastError();
}

}  // namespace gn
}  // namespace soar
