// model_ops.hip - the device operators of the SOAR model around the
// GroupNorm / convolution path: the general grouped convolution of the
// stem, sigmoid, channel-broadcast multiply, convex combination, global
// average pool, bilinear resize, pixel shuffle, spatial pad/crop, the
// Dice+BCE loss, and the multi-tensor gradient-norm / AdamW updates.
//
// Reference kernels (pomagrenate/soar.cpp): src/cuda/ops/
// convolution_kernels.cu (general conv2d), activation_kernels.cu (sigmoid),
// binary_ops_kernels.cu (mul_broadcast, convex_combination),
// pooling_kernels.cu (global_avg_pool), upsample_kernels.cu:11-135,
// loss_kernels.cu:29-265, optimizer_kernels.cu, and the host loops of
// src/nn/layers.cpp:807-1345, src/nn/soar_model.cpp:15-172,
// src/optim/adamw.cpp:28-108.
//
// All of these are small, HBM- or launch-bound passes.  Every reduction
// runs in a fixed order (per-thread sums, then a fixed-shape block tree,
// then a fixed-order finish), so results do not depend on scheduling; the
// reference's float atomics (loss_kernels.cu:46,131, upsample_kernels.cu:
// 97-100) are replaced by fp64 partials or by gathers.
#include "ops_internal.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace soar::ops {
namespace {

constexpr int kThreads = 256;

// Calls f with std::true_type or std::false_type: a runtime flag picks a
// kernel template instance.
template <typename F>
void bsel(bool b, F&& f) {
    if (b)
        f(std::true_type{});
    else
        f(std::false_type{});
}

int blocks_for(int64_t n, int64_t per_block = kThreads, int64_t cap = 8192) {
    int64_t b = (n + per_block - 1) / per_block;
    return (int)std::max<int64_t>(1, std::min<int64_t>(b, cap));
}

// Sum of `v` over a 256-thread block, the same tree every call; the result
// is valid in thread 0.
__device__ double block_sum(double v, double* sh) {
    const int t = threadIdx.x;
    sh[t] = v;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
        if (t < w) sh[t] += sh[t + w];
        __syncthreads();
    }
    const double r = sh[0];
    __syncthreads();  // sh may be reused as soon as this returns
    return r;
}

__device__ __forceinline__ float sigmoidf_exact(float z) { return 1.0f / (1.0f + expf(-z)); }

// Gradient store of the backward kernels: added (the reference's +=) or
// written, which saves the caller zeroing a fresh buffer.
template <bool ACC>
__device__ __forceinline__ void put(float* p, float v) {
    if (ACC)
        *p += v;
    else
        *p = v;
}

// ---------------------------------------------------------------------------
// General grouped convolution (convolution_kernels.cu conv2d_forward /
// conv2d_backward; layers.cpp:17-292 general branch).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_conv_fwd(const float* __restrict__ in,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ out, ConvShape c) {
    const int64_t total = c.N * c.C_out * c.Ho * c.Wo;
    const int64_t cig = c.C_in / c.groups, cog = c.C_out / c.groups;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t ox = i % c.Wo;
        int64_t t = i / c.Wo;
        const int64_t oy = t % c.Ho;
        t /= c.Ho;
        const int64_t co = t % c.C_out;
        const int64_t n = t / c.C_out;
        const int64_t ci0 = (co / cog) * cig;
        float acc = 0.0f;
        for (int64_t q = 0; q < cig; ++q) {
            const float* plane = in + ((n * c.C_in + ci0 + q) * c.H) * c.W;
            const float* wk = w + (co * cig + q) * c.K * c.K;
            for (int64_t ky = 0; ky < c.K; ++ky) {
                const int64_t iy = oy * c.S - c.pad + ky * c.D;
                if (iy < 0 || iy >= c.H) continue;
                for (int64_t kx = 0; kx < c.K; ++kx) {
                    const int64_t ix = ox * c.S - c.pad + kx * c.D;
                    if (ix < 0 || ix >= c.W) continue;
                    acc = fmaf(wk[ky * c.K + kx], plane[iy * c.W + ix], acc);
                }
            }
        }
        out[i] = bias ? acc + bias[co] : acc;
    }
}

// dx: every input element gathers the outputs its taps reach.
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_conv_dx(const float* __restrict__ go,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ gx, ConvShape c) {
    const int64_t total = c.N * c.C_in * c.H * c.W;
    const int64_t cig = c.C_in / c.groups, cog = c.C_out / c.groups;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t ix = i % c.W;
        int64_t t = i / c.W;
        const int64_t iy = t % c.H;
        t /= c.H;
        const int64_t ci = t % c.C_in;
        const int64_t n = t / c.C_in;
        const int64_t g = ci / cig, q = ci - g * cig;
        float acc = 0.0f;
        for (int64_t co = g * cog; co < (g + 1) * cog; ++co) {
            const float* gp = go + ((n * c.C_out + co) * c.Ho) * c.Wo;
            const float* wk = w + (co * cig + q) * c.K * c.K;
            for (int64_t ky = 0; ky < c.K; ++ky) {
                const int64_t ty = iy + c.pad - ky * c.D;
                if (ty < 0 || ty % c.S) continue;
                const int64_t oy = ty / c.S;
                if (oy >= c.Ho) continue;
                for (int64_t kx = 0; kx < c.K; ++kx) {
                    const int64_t tx = ix + c.pad - kx * c.D;
                    if (tx < 0 || tx % c.S) continue;
                    const int64_t ox = tx / c.S;
                    if (ox >= c.Wo) continue;
                    acc = fmaf(wk[ky * c.K + kx], gp[oy * c.Wo + ox], acc);
                }
            }
        }
        if (ACC)
            gx[i] += acc;
        else
            gx[i] = acc;
    }
}

constexpr int64_t kConvChunk = 16384;  // largest output-position chunk of a dW block
constexpr int kConvCoW = 4;            // output channels per wave of k_conv_dw_co

// Output positions per dW block: about 2048 blocks over the (co, q) rows
// and chunks, chunks of 1024..16384 positions (a thread walks its chunk's
// positions one after another, each a round of dependent loads), and at
// most 65535 chunks.
int64_t conv_chunk(const ConvShape& c) {
    const int64_t pos = c.N * c.Ho * c.Wo;
    const int64_t rows = std::max<int64_t>(1, c.C_out * (c.C_in / c.groups));
    const int64_t want = std::max<int64_t>(1, 2048 / rows);
    int64_t ch = (pos + want - 1) / want;
    ch = (ch + 1023) / 1024 * 1024;
    ch = std::max<int64_t>(1024, std::min<int64_t>(ch, kConvChunk));
    return std::max<int64_t>(ch, (pos + 65534) / 65535);
}

int64_t conv_chunks(const ConvShape& c) {
    const int64_t ch = conv_chunk(c);
    return (c.N * c.Ho * c.Wo + ch - 1) / ch;
}

// The dense few-channel kernels (k_conv_fwd_co / k_conv_dw_co) take the
// shape: one group, C_out a multiple of 4 up to 64, 32-bit positions.
bool conv_dense_small(const ConvShape& c) {
    return c.groups == 1 && c.C_out % kConvCoW == 0 && c.C_out <= 64 && c.C_in <= 64 &&
           c.N * c.Ho * c.Wo < ((int64_t)1 << 31) && c.H < ((int64_t)1 << 30) &&
           c.W < ((int64_t)1 << 30);
}

// Its weight gradient (K in {1, 3}): chunks of at least kConvDenseChunk
// positions, about 2048 blocks of 4 waves, at most 65535 chunks.  At the
// SOAR stem on 1024^2 (16 channels, 512^2 outputs) chunks of 256 / 512 /
// 1024 / 2048 positions took 36 / 24 / 28 / 48 us, and 2 positions per
// lane and step 24 us against 27 with 4.
#ifndef SOAR_CONV_DENSE_CHUNK
#define SOAR_CONV_DENSE_CHUNK 512
#endif
constexpr int64_t kConvDenseChunk = SOAR_CONV_DENSE_CHUNK;
#ifndef SOAR_CONV_DENSE_STEP
#define SOAR_CONV_DENSE_STEP 2
#endif
constexpr int kConvDenseStep = SOAR_CONV_DENSE_STEP;  // positions per lane per step
bool conv_dw_dense(const ConvShape& c) {
    return conv_dense_small(c) && (c.K == 1 || c.K == 3);
}

int64_t conv_dense_chunk(const ConvShape& c) {
    const int64_t pos = c.N * c.Ho * c.Wo;
    const int64_t waves = (c.C_out / kConvCoW) * c.C_in;
    const int64_t blocks_per_chunk = (waves + 3) / 4;
    const int64_t want = std::max<int64_t>(1, 2048 / blocks_per_chunk);
    int64_t ch = (pos + want - 1) / want;
    ch = std::max<int64_t>(kConvDenseChunk, (ch + 63) / 64 * 64);
    return std::max<int64_t>(ch, (pos + 65534) / 65535);
}

int64_t conv_dw_chunks(const ConvShape& c) {
    const int64_t ch = conv_dw_dense(c) ? conv_dense_chunk(c) : conv_chunk(c);
    return (c.N * c.Ho * c.Wo + ch - 1) / ch;
}

// dW / db partials: block x = (co*cig+q)*(K*K+1) + tap, block y = chunk;
// tap == K*K is the bias sum (only for q == 0).
// part[(co*cig+q)*(K*K+1)+tap][chunk].
__global__ __launch_bounds__(kThreads) void k_conv_dw(const float* __restrict__ go,
                                                      const float* __restrict__ in,
                                                      double* __restrict__ part, ConvShape c,
                                                      int64_t chunks, int64_t csize) {
    __shared__ double sh[kThreads];
    const int64_t chunk = blockIdx.y;
    const int64_t KK = c.K * c.K;
    const int64_t tap = (int64_t)blockIdx.x % (KK + 1);
    const int64_t cig = c.C_in / c.groups, cog = c.C_out / c.groups;
    const int64_t wq = (int64_t)blockIdx.x / (KK + 1);  // co*cig + q
    const int64_t co = wq / cig, q = wq - co * cig;
    const bool is_bias = tap == KK;
    double s = 0.0;
    if (!is_bias || q == 0) {
        const int64_t ci = (co / cog) * cig + q;
        const int64_t ky = is_bias ? 0 : tap / c.K, kx = is_bias ? 0 : tap % c.K;
        const int64_t HWo = c.Ho * c.Wo;
        const int64_t end = std::min((chunk + 1) * csize, c.N * HWo);
        for (int64_t p = chunk * csize + threadIdx.x; p < end; p += kThreads) {
            const int64_t n = p / HWo, r = p - n * HWo;
            const int64_t oy = r / c.Wo, ox = r - oy * c.Wo;
            const float g = go[(n * c.C_out + co) * HWo + r];
            if (is_bias) {
                s += g;
                continue;
            }
            const int64_t iy = oy * c.S - c.pad + ky * c.D;
            const int64_t ix = ox * c.S - c.pad + kx * c.D;
            if (iy < 0 || iy >= c.H || ix < 0 || ix >= c.W) continue;
            s += (double)g * in[((n * c.C_in + ci) * c.H + iy) * c.W + ix];
        }
    }
    s = block_sum(s, sh);
    if (threadIdx.x == 0) part[(wq * (KK + 1) + tap) * chunks + chunk] = s;
}

// The same partials for K in {1, 3, 5, 7}: one block computes all K*K tap
// sums and the bias sum of one (co, q) over one chunk, so the position
// arithmetic (32-bit: N*Ho*Wo < 2^31, checked by the host) and the dy load
// are shared by the taps.  Thread t walks positions t, t + 256, ... as
// above; the block adds its waves' trees in order.
template <int K>
__global__ __launch_bounds__(kThreads) void k_conv_dw_taps(const float* __restrict__ go,
                                                           const float* __restrict__ in,
                                                           double* __restrict__ part,
                                                           ConvShape c, int64_t chunks,
                                                           int64_t csize) {
    constexpr int KK = K * K, KK1 = KK + 1;
    __shared__ double red[kThreads / 64][KK1];
    const int64_t chunk = blockIdx.y;
    const int64_t wq = blockIdx.x;  // co*cig + q
    const int64_t cig = c.C_in / c.groups, cog = c.C_out / c.groups;
    const int64_t co = wq / cig, q = wq - co * cig;
    const int64_t ci = (co / cog) * cig + q;
    const uint32_t HWo = (uint32_t)(c.Ho * c.Wo), Wo = (uint32_t)c.Wo;
    const int H = (int)c.H, W = (int)c.W;
    const int S = (int)c.S, D = (int)c.D, pad = (int)c.pad;
    double sw[KK1];
#pragma unroll
    for (int k = 0; k < KK1; ++k) sw[k] = 0.0;
    const uint32_t p0 = (uint32_t)(chunk * csize);
    const uint32_t end = (uint32_t)std::min<int64_t>((chunk + 1) * csize, c.N * c.Ho * c.Wo);
    for (uint32_t p = p0 + threadIdx.x; p < end; p += kThreads) {
        const uint32_t n = p / HWo, r = p - n * HWo;
        const uint32_t oy = r / Wo, ox = r - oy * Wo;
        const float g = go[((int64_t)n * c.C_out + co) * HWo + r];
        sw[KK] += (double)g;
        const float* ip = in + ((int64_t)n * c.C_in + ci) * c.H * c.W;
        const int iy0 = (int)oy * S - pad, ix0 = (int)ox * S - pad;
#pragma unroll
        for (int ky = 0; ky < K; ++ky) {
            const int iy = iy0 + ky * D;
            if (iy < 0 || iy >= H) continue;
#pragma unroll
            for (int kx = 0; kx < K; ++kx) {
                const int ix = ix0 + kx * D;
                if (ix < 0 || ix >= W) continue;
                sw[ky * K + kx] += (double)g * ip[(int64_t)iy * W + ix];
            }
        }
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < KK1; ++k) {
        double v = sw[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off);
        if (lane == 0) red[wv][k] = v;
    }
    __syncthreads();
    for (int k = threadIdx.x; k < KK1; k += kThreads) {
        double v = red[0][k];
#pragma unroll
        for (int i = 1; i < kThreads / 64; ++i) v += red[i][k];
        part[(wq * KK1 + k) * chunks + chunk] = (k < KK || q == 0) ? v : 0.0;
    }
}

// Adds the chunk sums in order: gw[co][q][tap] += ..., gb[co] += ...
__global__ __launch_bounds__(kThreads) void k_conv_dw_finish(const double* __restrict__ part,
                                                             float* __restrict__ gw,
                                                             float* __restrict__ gb,
                                                             ConvShape c, int64_t chunks) {
    const int64_t KK = c.K * c.K;
    const int64_t cig = c.C_in / c.groups;
    const int64_t rows = c.C_out * cig * (KK + 1);
    for (int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x; r < rows;
         r += (int64_t)gridDim.x * kThreads) {
        const int64_t wq = r / (KK + 1), tap = r - wq * (KK + 1);
        const int64_t co = wq / cig, q = wq - co * cig;
        double s = 0.0;
        for (int64_t k = 0; k < chunks; ++k) s += part[r * chunks + k];
        if (tap < KK) {
            if (gw) gw[wq * KK + tap] += (float)s;
        } else if (q == 0 && gb) {
            gb[co] += (float)s;
        }
    }
}

// ---- dense convolutions with few output channels (SOAR's stem: 1 or 3
// input channels to 16, k3 stride 2, on the full-resolution image) -------
// The generic kernels above give every output channel its own thread and
// so read each input tap once per output channel (16 times at the stem),
// and the weight gradient's blocks do the same per (co, q) row.

// Forward: one thread per output position computes CT output channels from
// one read of its input taps.  Every output adds its taps in k_conv_fwd's
// order (input channel, ky, kx, taps outside the input skipped), so the
// values are k_conv_fwd's.  groups == 1, C_out % CT == 0, N*Ho*Wo < 2^31.
template <int CT>
__global__ __launch_bounds__(kThreads) void k_conv_fwd_co(const float* __restrict__ in,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ out, ConvShape c) {
    const uint32_t HWo = (uint32_t)(c.Ho * c.Wo), Wo = (uint32_t)c.Wo;
    const uint32_t P = (uint32_t)(c.N * c.Ho * c.Wo);
    const int H = (int)c.H, W = (int)c.W, K = (int)c.K, KK = K * K, cin = (int)c.C_in;
    const int S = (int)c.S, D = (int)c.D, pad = (int)c.pad;
    const int64_t co0 = (int64_t)blockIdx.y * CT;
    const uint32_t p = blockIdx.x * kThreads + threadIdx.x;  // one position per thread
    if (p < P) {
        const uint32_t n = p / HWo, r = p - n * HWo;
        const uint32_t oy = r / Wo, ox = r - oy * Wo;
        const int iy0 = (int)oy * S - pad, ix0 = (int)ox * S - pad;
        float acc[CT];
#pragma unroll
        for (int j = 0; j < CT; ++j) acc[j] = 0.0f;
        for (int q = 0; q < cin; ++q) {
            const float* plane = in + ((int64_t)n * cin + q) * c.H * c.W;
            const float* wq = w + (co0 * cin + q) * KK;  // + j * cin * KK: channel co0 + j
            for (int ky = 0; ky < K; ++ky) {
                const int iy = iy0 + ky * D;
                if (iy < 0 || iy >= H) continue;
                for (int kx = 0; kx < K; ++kx) {
                    const int ix = ix0 + kx * D;
                    if (ix < 0 || ix >= W) continue;
                    const float x = plane[(int64_t)iy * W + ix];
#pragma unroll
                    for (int j = 0; j < CT; ++j)
                        acc[j] = fmaf(wq[(int64_t)j * cin * KK + ky * K + kx], x, acc[j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            float* o = out + ((int64_t)n * c.C_out + co0 + j) * HWo + r;
            *o = bias ? acc[j] + bias[co0 + j] : acc[j];
        }
    }
}

// dW / db partials with a wave per (kConvCoW = 4 output channels, input
// channel q): its lanes walk positions p0 + lane, p0 + lane + 64, ... of
// the chunk, read dy of the 4 channels and the K*K input taps once per
// position (taps outside the input read as zero), and keep the
// 4 x (K*K + 1) sums in float64; the wave adds its lanes in a fixed tree.
// Same partial layout as k_conv_dw_taps (one per chunk).  groups == 1,
// C_out % 4 == 0, K in {1, 3}, 32-bit position arithmetic.
template <int K>
__global__ __launch_bounds__(kThreads) void k_conv_dw_co(const float* __restrict__ go,
                                                         const float* __restrict__ in,
                                                         double* __restrict__ part, ConvShape c,
                                                         int64_t chunks, int64_t csize) {
    constexpr int KK = K * K, KK1 = KK + 1;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t cin = c.C_in;
    const int64_t task = (int64_t)blockIdx.x * (kThreads / 64) + wv;  // (channel group, q)
    if (task >= (c.C_out / kConvCoW) * cin) return;  // (no block barrier below)
    const int64_t co0 = task / cin * kConvCoW, q = task % cin;
    const uint32_t HWo = (uint32_t)(c.Ho * c.Wo), Wo = (uint32_t)c.Wo;
    const int H = (int)c.H, W = (int)c.W;
    const int S = (int)c.S, D = (int)c.D, pad = (int)c.pad;
    const uint32_t chunk = blockIdx.y;
    const uint32_t p0 = (uint32_t)(chunk * csize);
    const uint32_t end = (uint32_t)std::min<int64_t>((chunk + 1) * csize, c.N * c.Ho * c.Wo);
    double acc[kConvCoW][KK1];
#pragma unroll
    for (int j = 0; j < kConvCoW; ++j)
#pragma unroll
        for (int k = 0; k < KK1; ++k) acc[j][k] = 0.0;
    // kConvDenseStep positions per step (p, p + 64, ...), their loads
    // issued together; the sums take them in position order
    auto load = [&](uint32_t p, float* g, float* x) {
        const uint32_t n = p / HWo, r = p - n * HWo;
        const uint32_t oy = r / Wo, ox = r - oy * Wo;
#pragma unroll
        for (int j = 0; j < kConvCoW; ++j) g[j] = go[((int64_t)n * c.C_out + co0 + j) * HWo + r];
        const float* ip = in + ((int64_t)n * cin + q) * c.H * c.W;
        const int iy0 = (int)oy * S - pad, ix0 = (int)ox * S - pad;
#pragma unroll
        for (int ky = 0; ky < K; ++ky)
#pragma unroll
            for (int kx = 0; kx < K; ++kx) {
                const int iy = iy0 + ky * D, ix = ix0 + kx * D;
                const bool inside = iy >= 0 && iy < H && ix >= 0 && ix < W;
                x[ky * K + kx] = inside ? ip[(int64_t)iy * W + ix] : 0.0f;
            }
    };
    auto add = [&](const float* g, const float* x) {
#pragma unroll
        for (int j = 0; j < kConvCoW; ++j) {
            acc[j][KK] += (double)g[j];
#pragma unroll
            for (int k = 0; k < KK; ++k) acc[j][k] += (double)g[j] * (double)x[k];
        }
    };
    for (uint32_t p = p0 + lane; p < end; p += 64 * kConvDenseStep) {
        float g[kConvDenseStep][kConvCoW], x[kConvDenseStep][KK];
#pragma unroll
        for (int i = 0; i < kConvDenseStep; ++i)
            if (p + 64 * i < end) load(p + 64 * i, g[i], x[i]);
#pragma unroll
        for (int i = 0; i < kConvDenseStep; ++i)
            if (p + 64 * i < end) add(g[i], x[i]);
    }
#pragma unroll
    for (int j = 0; j < kConvCoW; ++j)
#pragma unroll
        for (int k = 0; k < KK1; ++k) {
            double v = acc[j][k];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off);
            if (lane == 0)
                part[(((co0 + j) * cin + q) * KK1 + k) * chunks + chunk] =
                    (k < KK || q == 0) ? v : 0.0;
        }
}

// k_conv_dw_finish with a wave per row: lane l adds chunks l, l + 64, ...
// in order, then the wave's fixed tree; for many chunks.
__global__ __launch_bounds__(kThreads) void k_conv_dw_finish_wave(
    const double* __restrict__ part, float* __restrict__ gw, float* __restrict__ gb,
    ConvShape c, int64_t chunks) {
    const int64_t KK = c.K * c.K;
    const int64_t cig = c.C_in / c.groups;
    const int64_t rows = c.C_out * cig * (KK + 1);
    const int64_t r = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    double s = 0.0;
    for (int64_t k = lane; k < chunks; k += 64) s += part[r * chunks + k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_down(s, off);
    if (lane != 0) return;
    const int64_t wq = r / (KK + 1), tap = r - wq * (KK + 1);
    const int64_t co = wq / cig, q = wq - co * cig;
    if (tap < KK) {
        if (gw) gw[wq * KK + tap] += (float)s;
    } else if (q == 0 && gb) {
        gb[co] += (float)s;
    }
}

// ---------------------------------------------------------------------------
// Elementwise operators.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_sigmoid_fwd(const float* __restrict__ x,
                                                          float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads)
        y[i] = sigmoidf_exact(x[i]);
}

// gx += gy * y * (1 - y)   (activation_kernels.cu:173, layers.cpp:826-831)
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_sigmoid_bwd(const float* __restrict__ gy,
                                                          const float* __restrict__ y,
                                                          float* __restrict__ gx, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float v = y[i];
        put<ACC>(gx + i, gy[i] * v * (1.0f - v));
    }
}

__global__ __launch_bounds__(kThreads) void k_mul_bcast_fwd(const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            float* __restrict__ y, int64_t rows,
                                                            int64_t HW) {
    const int64_t n = rows * HW;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads)
        y[i] = a[i] * b[i / HW];
}

// ga += gy * b[row]; gb[row] += sum gy*a (one block per row; the
// reference's per-element atomicAdd, binary_ops_kernels.cu:129, becomes a
// fixed-order block sum).
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_mul_bcast_bwd(const float* __restrict__ gy,
                                                            const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            float* __restrict__ ga,
                                                            float* __restrict__ gb, int64_t HW) {
    __shared__ double sh[kThreads];
    const int64_t row = blockIdx.x;
    const float* g = gy + row * HW;
    const float* ar = a + row * HW;
    const float bv = b[row];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < HW; i += kThreads) {
        const float gv = g[i];
        if (ga) put<ACC>(ga + row * HW + i, gv * bv);
        if (gb) s += (double)gv * ar[i];
    }
    if (gb) {
        s = block_sum(s, sh);
        if (threadIdx.x == 0) put<ACC>(gb + row, (float)s);
    }
}

// y = g*a + (1-g)*b   (blocks.cpp:333)
__global__ __launch_bounds__(kThreads) void k_convex_fwd(const float* __restrict__ g,
                                                         const float* __restrict__ a,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float gv = g[i];
        y[i] = gv * a[i] + (1.0f - gv) * b[i];
    }
}

template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_convex_bwd(const float* __restrict__ gy,
                                                         const float* __restrict__ g,
                                                         const float* __restrict__ a,
                                                         const float* __restrict__ b,
                                                         float* __restrict__ gg,
                                                         float* __restrict__ ga,
                                                         float* __restrict__ gb, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float d = gy[i], gv = g[i];
        if (ga) put<ACC>(ga + i, d * gv);
        if (gb) put<ACC>(gb + i, d * (1.0f - gv));
        if (gg) put<ACC>(gg + i, d * (a[i] - b[i]));
    }
}

// ---- the SOAR gates with their sigmoid folded in --------------------------
// Fuse (blocks.cpp:333): y = s*a + (1-s)*b with s = sigmoid(z), and Ctx:
// y[c][i] = a[c][i] * sigmoid(z[c]).  s is recomputed from z wherever it is
// needed (sigmoidf_exact, the sigmoid kernel's own arithmetic), so the
// values, and the gradients below, are those of the sigmoid kernel followed
// by the convex-combination / broadcast-multiply kernel, one launch each
// direction instead of two.
__global__ __launch_bounds__(kThreads) void k_sigmoid_convex_fwd(const float* __restrict__ z,
                                                                 const float* __restrict__ a,
                                                                 const float* __restrict__ b,
                                                                 float* __restrict__ y,
                                                                 int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float gv = sigmoidf_exact(z[i]);
        y[i] = gv * a[i] + (1.0f - gv) * b[i];
    }
}

// ga = gy*s, gb = gy*(1-s), gz = (gy*(a-b)) * s * (1-s)
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_sigmoid_convex_bwd(
    const float* __restrict__ gy, const float* __restrict__ z, const float* __restrict__ a,
    const float* __restrict__ b, float* __restrict__ gz, float* __restrict__ ga,
    float* __restrict__ gb, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float d = gy[i], gv = sigmoidf_exact(z[i]);
        if (ga) put<ACC>(ga + i, d * gv);
        if (gb) put<ACC>(gb + i, d * (1.0f - gv));
        if (gz) {
            const float gg = d * (a[i] - b[i]);
            put<ACC>(gz + i, gg * gv * (1.0f - gv));
        }
    }
}

__global__ __launch_bounds__(kThreads) void k_mul_sigmoid_fwd(const float* __restrict__ a,
                                                              const float* __restrict__ z,
                                                              float* __restrict__ y,
                                                              int64_t rows, int64_t HW) {
    const int64_t n = rows * HW;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads)
        y[i] = a[i] * sigmoidf_exact(z[i / HW]);
}

// ga = gy * s[row]; gz[row] = (float)(sum gy*a) * s * (1-s), one block per row
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_mul_sigmoid_bwd(const float* __restrict__ gy,
                                                              const float* __restrict__ a,
                                                              const float* __restrict__ z,
                                                              float* __restrict__ ga,
                                                              float* __restrict__ gz,
                                                              int64_t HW) {
    __shared__ double sh[kThreads];
    const int64_t row = blockIdx.x;
    const float* g = gy + row * HW;
    const float* ar = a + row * HW;
    const float bv = sigmoidf_exact(z[row]);
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < HW; i += kThreads) {
        const float gv = g[i];
        if (ga) put<ACC>(ga + row * HW + i, gv * bv);
        if (gz) s += (double)gv * ar[i];
    }
    if (gz) {
        s = block_sum(s, sh);
        if (threadIdx.x == 0) {
            const float gb = (float)s;
            put<ACC>(gz + row, gb * bv * (1.0f - bv));
        }
    }
}

// ---------------------------------------------------------------------------
// Global average pool: one block per plane (layers.cpp:1306-1345).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void k_avg_pool_fwd(const float* __restrict__ in,
                                                           float* __restrict__ out, int64_t HW) {
    __shared__ double sh[kThreads];
    const float* p = in + (int64_t)blockIdx.x * HW;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < HW; i += kThreads) s += p[i];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) out[blockIdx.x] = (float)(s / (double)HW);
}

// gi += go[row] / HW   (pooling_kernels.cu:27-33)
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_avg_pool_bwd(const float* __restrict__ go,
                                                           float* __restrict__ gi, int64_t rows,
                                                           int64_t HW) {
    const int64_t n = rows * HW;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads)
        put<ACC>(gi + i, go[i / HW] / (float)HW);
}

// ---------------------------------------------------------------------------
// Bilinear resize, half-pixel centres, no corner alignment
// (upsample_kernels.cu:11-66, layers.cpp:1073-1150).
// ---------------------------------------------------------------------------
struct Src {
    int i0, i1;    // the two source taps (equal at the last row / column)
    float l0, l1;  // their weights
};

// (plane sides are below 2^31: the C-ABI checks them)
__device__ __forceinline__ Src src_index(float scale, int dst, int n_in) {
    float r = scale * ((float)dst + 0.5f) - 0.5f;
    r = r < 0.0f ? 0.0f : r;
    const int i0 = min((int)r, n_in - 1);
    const int step = i0 < n_in - 1 ? 1 : 0;
    const float l1 = r - (float)i0;
    return {i0, i0 + step, 1.0f - l1, l1};
}

// Element indices have type I (32-bit when both tensors' element counts
// fit: the index arithmetic is most of this kernel's instructions).
template <typename I>
__global__ __launch_bounds__(kThreads) void k_upsample_fwd(const float* __restrict__ in,
                                                           float* __restrict__ out, I rows,
                                                           I H_in, I W_in, I H_out, I W_out,
                                                           float sh, float sw) {
    const I total = rows * H_out * W_out;
    for (I i = (I)blockIdx.x * kThreads + threadIdx.x; i < total; i += (I)gridDim.x * kThreads) {
        const I x = i % W_out;
        const I t = i / W_out;
        const I y = t % H_out;
        const I row = t / H_out;
        const Src sy = src_index(sh, (int)y, (int)H_in), sx = src_index(sw, (int)x, (int)W_in);
        const float* p = in + (int64_t)row * H_in * W_in;
        const float v00 = p[(I)sy.i0 * W_in + sx.i0], v01 = p[(I)sy.i0 * W_in + sx.i1];
        const float v10 = p[(I)sy.i1 * W_in + sx.i0], v11 = p[(I)sy.i1 * W_in + sx.i1];
        out[i] = sy.l0 * (sx.l0 * v00 + sx.l1 * v01) + sy.l1 * (sx.l0 * v10 + sx.l1 * v11);
    }
}

// Destinations along one axis whose taps reach source index `s`.  They form
// one contiguous run: a destination's first tap is non-decreasing in the
// destination index, and of the destinations whose first tap is s - 1 only
// the first can give s a zero weight.  The run is found inside a candidate
// window that is conservative by one on each side.  Returns the run length
// (0 when no destination reads s, as when downsampling) and its first index.
__device__ __forceinline__ void dst_window(float scale, int s, int n_out, int* lo, int* hi) {
    // both bounds are non-decreasing in s
    const float a = ((float)s - 0.5f) / scale - 0.5f;
    const float b = ((float)s + 1.5f) / scale - 0.5f;
    *lo = max(0, (int)floorf(a) - 1);
    *hi = min(n_out - 1, (int)ceilf(b) + 1);
}

__device__ __forceinline__ int dst_run(float scale, int s, int n_in, int n_out, int* first) {
    int d, hi;
    dst_window(scale, s, n_out, &d, &hi);
    auto w = [&](int i) {
        const Src t = src_index(scale, i, n_in);
        return (t.i0 == s ? t.l0 : 0.0f) + (t.i1 == s ? t.l1 : 0.0f);
    };
    while (d <= hi && w(d) == 0.0f) ++d;
    int n = 0;
    while (d + n <= hi && w(d + n) != 0.0f) ++n;
    *first = d;
    return n;
}

__device__ __forceinline__ float tap_weight(const Src& s, int idx) {
    return (s.i0 == idx ? s.l0 : 0.0f) + (s.i1 == idx ? s.l1 : 0.0f);
}

// Backward as a gather: each source pixel sums the destination pixels that
// read it, with the forward's weights, rows in order and within a row
// columns in order (no atomics).  The column weights of a run of at most R
// destinations are computed once and kept in registers, and each row's R
// loads are issued together (clamped to the run, the extra lanes weighted
// out); longer runs take the plain loop.  Element indices have type I
// (32-bit when both tensors' element counts fit); plane sides fit in int.
template <int R>
__device__ float gather_one(const float* __restrict__ g, int iy, int ix, int H_in, int W_in,
                            int H_out, int W_out, float sh, float sw) {
    int ya, xa;
    const int ny = dst_run(sh, iy, H_in, H_out, &ya);
    const int nx = dst_run(sw, ix, W_in, W_out, &xa);
    float acc = 0.0f;
    if (nx > 0 && nx <= R) {  // (a zero-length run may start past the row)
        float wx[R];
#pragma unroll
        for (int j = 0; j < R; ++j)
            wx[j] = j < nx ? tap_weight(src_index(sw, xa + j, W_in), ix) : 0.0f;
        const int xl = xa + nx - 1;
        for (int k = 0; k < ny; ++k) {
            const int y = ya + k;
            const float wy = tap_weight(src_index(sh, y, H_in), iy);
            const float* gr = g + (int64_t)y * W_out;
            float v[R];
#pragma unroll
            for (int j = 0; j < R; ++j) v[j] = gr[min(xa + j, xl)];
            float rs = 0.0f;
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (j < nx) rs += wx[j] * v[j];
            acc += wy * rs;
        }
    } else {
        for (int k = 0; k < ny; ++k) {
            const int y = ya + k;
            const float wy = tap_weight(src_index(sh, y, H_in), iy);
            const float* gr = g + (int64_t)y * W_out;
            float rs = 0.0f;
            for (int j = 0; j < nx; ++j)
                rs += tap_weight(src_index(sw, xa + j, W_in), ix) * gr[xa + j];
            acc += wy * rs;
        }
    }
    return acc;
}

template <int R, typename I, bool ACC>
__global__ __launch_bounds__(kThreads) void k_upsample_bwd(const float* __restrict__ go,
                                                           float* __restrict__ gi, I rows,
                                                           int H_in, int W_in, int H_out,
                                                           int W_out, float sh, float sw) {
    const I total = rows * H_in * W_in;
    for (I i = (I)blockIdx.x * kThreads + threadIdx.x; i < total; i += (I)gridDim.x * kThreads) {
        const int ix = (int)(i % W_in);
        const I t = i / W_in;
        const int iy = (int)(t % H_in);
        const I row = t / H_in;
        put<ACC>(gi + i, gather_one<R>(go + (int64_t)row * H_out * W_out, iy, ix, H_in, W_in,
                                       H_out, W_out, sh, sw));
    }
}

// Backward for exact integer factors F (2 or 4) on both axes: every
// destination that reads source s lies in [F s - F/2, F s + 3F/2 - 1], 2F
// candidates per axis, so the taps need no search (checked against every
// destination for sides up to 299; the sides are capped at 2^22, where the
// fp32 source coordinates are exact).  Zero-weight candidates are skipped,
// so the terms and their order are gather_one's and the results identical.
template <int F, typename I, bool ACC>
__global__ __launch_bounds__(kThreads) void k_upsample_bwd_int(const float* __restrict__ go,
                                                               float* __restrict__ gi, I rows,
                                                               int H_in, int W_in, float sh,
                                                               float sw) {
    constexpr int NC = 2 * F, OFF = F / 2;
    const int H_out = F * H_in, W_out = F * W_in;
    const I total = rows * H_in * W_in;
    for (I i = (I)blockIdx.x * kThreads + threadIdx.x; i < total; i += (I)gridDim.x * kThreads) {
        const int ix = (int)(i % W_in);
        const I t = i / W_in;
        const int iy = (int)(t % H_in);
        const I row = t / H_in;
        const float* g = go + (int64_t)row * H_out * W_out;
        float wx[NC];
        int xs[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int x = F * ix - OFF + j;
            const bool in = x >= 0 && x < W_out;
            wx[j] = in ? tap_weight(src_index(sw, x, W_in), ix) : 0.0f;
            xs[j] = in ? x : 0;
        }
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            const int y = F * iy - OFF + k;
            if (y < 0 || y >= H_out) continue;
            const float wy = tap_weight(src_index(sh, y, H_in), iy);
            if (wy == 0.0f) continue;
            const float* gr = g + (int64_t)y * W_out;
            float v[NC];
#pragma unroll
            for (int j = 0; j < NC; ++j) v[j] = gr[xs[j]];
            float rs = 0.0f;
#pragma unroll
            for (int j = 0; j < NC; ++j)
                if (wx[j] != 0.0f) rs += wx[j] * v[j];
            acc += wy * rs;
        }
        put<ACC>(gi + i, acc);
    }
}

// Tiled backward for resizes by at most about 2x (or 4x) per axis.  A block
// owns TY x 64 source pixels of one plane.  It stages the window of
// destination rows and columns whose taps can reach them in LDS (coalesced
// loads: each destination value is read from memory about once, against
// once per tap in the per-pixel kernel), sums each window row over every
// source column's run of destination columns, then each source pixel sums
// its run of those row sums.  The terms and their order are the per-pixel
// kernel's (columns in order within a row, then rows in order), so both
// kernels give identical results.  A window larger than the LDS arrays
// (not expected for the factors the host routes here) makes that tile
// gather from global memory instead.
template <int TY, int WR, int WC, int R, bool ACC>
__global__ __launch_bounds__(kThreads) void k_upsample_bwd_tiled(
    const float* __restrict__ go, float* __restrict__ gi, int64_t rows, int H_in, int W_in,
    int H_out, int W_out, float sh, float sw, int tiles_y, int tiles_x) {
    static_assert(kThreads % 64 == 0, "a thread keeps one source column");
    constexpr int kRowStep = kThreads / 64;
    __shared__ float win[WR][WC + 1];
    __shared__ float rsum[WR][64];
    const int c = threadIdx.x & 63;       // this thread's source column in the tile
    const int r0 = threadIdx.x >> 6;      // and its first row (then every kRowStep-th)
    const int64_t ntiles = rows * tiles_y * tiles_x;
    for (int64_t b = blockIdx.x; b < ntiles; b += gridDim.x) {
        const int tx = (int)(b % tiles_x);
        const int64_t q = b / tiles_x;
        const int ty = (int)(q % tiles_y);
        const int64_t row = q / tiles_y;
        const int iy0 = ty * TY, ix0 = tx * 64;
        const int iy1 = min(iy0 + TY, H_in) - 1, ix1 = min(ix0 + 64, W_in) - 1;
        int ylo, yhi, xlo, xhi, unused;
        dst_window(sh, iy0, H_out, &ylo, &unused);
        dst_window(sh, iy1, H_out, &unused, &yhi);
        dst_window(sw, ix0, W_out, &xlo, &unused);
        dst_window(sw, ix1, W_out, &unused, &xhi);
        const int nr = yhi - ylo + 1, nc = xhi - xlo + 1;
        const float* g = go + row * H_out * W_out;
        float* gp = gi + row * H_in * W_in;
        const int ix = ix0 + c;
        if (nr > WR || nc > WC) {  // block-uniform
            for (int rr = r0; rr < TY; rr += kRowStep) {
                const int iy = iy0 + rr;
                if (iy <= iy1 && ix <= ix1)
                    put<ACC>(gp + (int64_t)iy * W_in + ix,
                             gather_one<R>(g, iy, ix, H_in, W_in, H_out, W_out, sh, sw));
            }
            continue;
        }
        {
            // wave w stages rows w, w + kRowStep, ...; lane l columns l, l + 64,
            // ...: every load is issued before the first LDS store
            constexpr int kRows = (WR + kRowStep - 1) / kRowStep, kCols = (WC + 63) / 64;
            float v[kRows][kCols];
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
                const int rr = r0 + i * kRowStep;
                const float* src = g + (int64_t)(ylo + min(rr, nr - 1)) * W_out + xlo;
#pragma unroll
                for (int j = 0; j < kCols; ++j) v[i][j] = src[min(c + 64 * j, nc - 1)];
            }
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
                const int rr = r0 + i * kRowStep;
#pragma unroll
                for (int j = 0; j < kCols; ++j)
                    if (rr < nr && c + 64 * j < nc) win[rr][c + 64 * j] = v[i][j];
            }
        }
        __syncthreads();
        // this column's run of destination columns, inside [xlo, xhi]
        int xa = 0, nx = 0;
        if (ix <= ix1) nx = dst_run(sw, ix, W_in, W_out, &xa);
        xa -= xlo;
        if (nx > 0 && nx <= R) {
            float wx[R];
#pragma unroll
            for (int j = 0; j < R; ++j)
                wx[j] = j < nx ? tap_weight(src_index(sw, xlo + xa + j, W_in), ix) : 0.0f;
            const int xl = xa + nx - 1;
            for (int rr = r0; rr < nr; rr += kRowStep) {
                float rs = 0.0f;
#pragma unroll
                for (int j = 0; j < R; ++j) {
                    const float v = win[rr][min(xa + j, xl)];
                    if (j < nx) rs += wx[j] * v;
                }
                rsum[rr][c] = rs;
            }
        } else {
            for (int rr = r0; rr < nr; rr += kRowStep) {
                float rs = 0.0f;
                for (int j = 0; j < nx; ++j)
                    rs += tap_weight(src_index(sw, xlo + xa + j, W_in), ix) * win[rr][xa + j];
                rsum[rr][c] = rs;
            }
        }
        __syncthreads();
        for (int rr = r0; rr < TY; rr += kRowStep) {
            const int iy = iy0 + rr;
            if (iy > iy1 || ix > ix1) continue;
            int ya;
            const int ny = dst_run(sh, iy, H_in, H_out, &ya);
            float acc = 0.0f;
            for (int k = 0; k < ny; ++k)
                acc += tap_weight(src_index(sh, ya + k, H_in), iy) * rsum[ya + k - ylo][c];
            put<ACC>(gp + (int64_t)iy * W_in + ix, acc);
        }
        __syncthreads();  // win and rsum are refilled for the next tile
    }
}

// ---------------------------------------------------------------------------
// Pixel shuffle (layers.cpp:928-989): out[c][y][x] =
// in[c*r*r + (y%r)*r + x%r][y/r][x/r]; the backward adds each output
// gradient to the input element it came from (a permutation, no
// collisions).
// ---------------------------------------------------------------------------
template <bool BWD, bool ACC>
__global__ __launch_bounds__(kThreads) void k_pixel_shuffle(const float* __restrict__ src,
                                                            float* __restrict__ dst, int64_t N,
                                                            int64_t C_out, int64_t H_in,
                                                            int64_t W_in, int64_t r) {
    const int64_t H_out = H_in * r, W_out = W_in * r;
    const int64_t total = N * C_out * H_out * W_out;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t x = i % W_out;
        int64_t t = i / W_out;
        const int64_t y = t % H_out;
        t /= H_out;  // n*C_out + c
        const int64_t cin = t * r * r + (y % r) * r + (x % r);
        const int64_t j = (cin * H_in + y / r) * W_in + x / r;
        if (BWD)
            put<ACC>(dst + j, src[i]);
        else
            dst[i] = src[j];
    }
}

// ---------------------------------------------------------------------------
// Spatial pad to a multiple of the model stride (soar_model.cpp:74-135):
// rows past H (columns past W) copy the reflected row 2(H-1)-y, or the last
// row when the pad is not smaller than the image.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t pad_src(int64_t y, int64_t H, bool reflect) {
    return y < H ? y : (reflect ? 2 * (H - 1) - y : H - 1);
}

__global__ __launch_bounds__(kThreads) void k_pad_fwd(const float* __restrict__ in,
                                                      float* __restrict__ out, int64_t rows,
                                                      int64_t H, int64_t W, int64_t Hp,
                                                      int64_t Wp, bool reflect) {
    const int64_t total = rows * Hp * Wp;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t x = i % Wp;
        int64_t t = i / Wp;
        const int64_t y = t % Hp;
        const int64_t row = t / Hp;
        out[i] = in[(row * H + pad_src(y, H, reflect)) * W + pad_src(x, W, reflect)];
    }
}

// Padded rows that read source row `s`: s itself plus, when reflecting,
// 2(H-1)-s if it lies in [H, Hp); when clamping, every row >= H for s=H-1.
__device__ __forceinline__ int pad_dsts(int64_t s, int64_t H, int64_t Hp, bool reflect,
                                        int64_t* first, int64_t* extra_lo, int64_t* extra_hi) {
    *first = s;
    *extra_lo = 1;
    *extra_hi = 0;  // empty range
    if (reflect) {
        const int64_t d = 2 * (H - 1) - s;
        if (d >= H && d < Hp) *extra_lo = *extra_hi = d;
    } else if (s == H - 1 && Hp > H) {
        *extra_lo = H;
        *extra_hi = Hp - 1;
    }
    return 0;
}

__global__ __launch_bounds__(kThreads) void k_pad_bwd(const float* __restrict__ go,
                                                      float* __restrict__ gi, int64_t rows,
                                                      int64_t H, int64_t W, int64_t Hp,
                                                      int64_t Wp, bool reflect) {
    const int64_t total = rows * H * W;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t x = i % W;
        int64_t t = i / W;
        const int64_t y = t % H;
        const int64_t row = t / H;
        int64_t fy, ylo, yhi, fx, xlo, xhi;
        pad_dsts(y, H, Hp, reflect, &fy, &ylo, &yhi);
        pad_dsts(x, W, Wp, reflect, &fx, &xlo, &xhi);
        const float* g = go + row * Hp * Wp;
        auto row_sum = [&](int64_t yy) {
            float s = g[yy * Wp + fx];
            for (int64_t xx = xlo; xx <= xhi; ++xx) s += g[yy * Wp + xx];
            return s;
        };
        float acc = row_sum(fy);
        for (int64_t yy = ylo; yy <= yhi; ++yy) acc += row_sum(yy);
        gi[i] += acc;
    }
}

template <bool BWD>
__global__ __launch_bounds__(kThreads) void k_crop(const float* __restrict__ src,
                                                   float* __restrict__ dst, int64_t rows,
                                                   int64_t Hp, int64_t Wp, int64_t H,
                                                   int64_t W) {
    // forward: dst [rows][H][W] from src [rows][Hp][Wp];
    // backward: dst [rows][Hp][Wp] += src [rows][H][W] (nothing outside).
    const int64_t total = BWD ? rows * Hp * Wp : rows * H * W;
    const int64_t ow = BWD ? Wp : W, oh = BWD ? Hp : H;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t x = i % ow;
        int64_t t = i / ow;
        const int64_t y = t % oh;
        const int64_t row = t / oh;
        if (BWD)
            dst[i] += (y < H && x < W) ? src[(row * H + y) * W + x] : 0.0f;
        else
            dst[i] = src[(row * Hp + y) * Wp + x];
    }
}

// ---------------------------------------------------------------------------
// Dice + BCE loss (loss_kernels.cu:29-265; losses.cpp:80-122,207-262).
// ---------------------------------------------------------------------------
constexpr int kLossBlocks = 1024;

__global__ __launch_bounds__(kThreads) void k_loss_sums(const float* __restrict__ z,
                                                        const float* __restrict__ y, int64_t n,
                                                        float pos_weight,
                                                        double* __restrict__ part) {
    __shared__ double sh[kThreads];
    double bce = 0.0, inter = 0.0, sp = 0.0, sy = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float zi = z[i], yi = y[i];
        const float w = 1.0f + (pos_weight - 1.0f) * yi;
        const float term = fmaxf(-zi, 0.0f) + log1pf(expf(-fabsf(zi)));
        bce += (double)((1.0f - yi) * zi + w * term);
        const float p = sigmoidf_exact(zi);
        inter += (double)(p * yi);
        sp += p;
        sy += yi;
    }
    const double v[4] = {bce, inter, sp, sy};
    for (int k = 0; k < 4; ++k) {
        const double s = block_sum(v[k], sh);
        if (threadIdx.x == 0) part[k * gridDim.x + blockIdx.x] = s;
    }
}

__global__ __launch_bounds__(kThreads) void k_loss_finish(const double* __restrict__ part,
                                                          int nparts, double* __restrict__ out) {
    // per quantity: thread t adds blocks t, t + kThreads, ... in order, then
    // the fixed block tree (a lone thread walking 1024 partials took 80 us)
    __shared__ double sh[kThreads];
    for (int k = 0; k < 4; ++k) {
        double v = 0.0;
        for (int b = threadIdx.x; b < nparts; b += kThreads) v += part[k * nparts + b];
        const double s = block_sum(v, sh);
        if (threadIdx.x == 0) out[k] = s;
    }
}

// Dice terms from the loss sums (inter, sum_p, sum_y handed on as fp32, as
// the host finish does), rounded as the host evaluates them.
__device__ __forceinline__ void dice_terms(const double* __restrict__ sums, float smooth,
                                           float* denom, float* numer) {
#pragma clang fp contract(off)
    const float inter = (float)sums[1], sum_p = (float)sums[2], sum_y = (float)sums[3];
    *denom = sum_p + sum_y + smooth;
    *numer = 2.0f * inter + smooth;
}

// gz += BCE gradient * scale_bce + Dice gradient * scale_dice
// (loss_kernels.cu:212-252; losses.cpp:497-541).  sums (device, optional):
// denom and numer come from the loss sums there instead of the arguments.
template <bool ACC>
__global__ __launch_bounds__(kThreads) void k_dice_bce_bwd(const float* __restrict__ z,
                                                           const float* __restrict__ y,
                                                           float* __restrict__ gz, int64_t n,
                                                           float scale_bce, float scale_dice,
                                                           float pos_weight, float denom,
                                                           float numer, float smooth,
                                                           const double* __restrict__ sums) {
    if (sums) dice_terms(sums, smooth, &denom, &numer);
    const float denom_sq = denom * denom;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float zi = z[i], yi = y[i];
        const float sig = sigmoidf_exact(zi);
        float g = 0.0f;
        if (scale_bce != 0.0f) {
            const float w_pos = 1.0f + (pos_weight - 1.0f) * yi;
            g += (sig * w_pos - pos_weight * yi) * scale_bce;
        }
        if (scale_dice != 0.0f) {
            const float dp_dz = sig * (1.0f - sig);
            const float d_dice_dp = (2.0f * yi * denom - numer) / denom_sq;
            g += scale_dice * (-d_dice_dp * dp_dz);
        }
        put<ACC>(gz + i, g);
    }
}

__global__ __launch_bounds__(kThreads) void k_sigmoid_threshold(const float* __restrict__ z,
                                                                float* __restrict__ p,
                                                                uint8_t* __restrict__ mask,
                                                                int64_t n, float threshold) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * kThreads) {
        const float v = sigmoidf_exact(z[i]);
        if (p) p[i] = v;
        if (mask) mask[i] = v >= threshold ? 1 : 0;
    }
}

// ---------------------------------------------------------------------------
// Channel concatenation of K tensors [N][C_k][HW] into [N][sum C_k][HW] and
// its backward, one launch for every (sample, piece) copy (the reference
// issues one copy per piece and sample, blocks.cpp concat_channels).  Block
// row y takes the pieces y, y + gridDim.y, ... of the N*K (sample, piece)
// pairs; its blocks stride over that piece's C_k*HW contiguous floats.
// ---------------------------------------------------------------------------
template <int V, bool BWD>
__global__ __launch_bounds__(kThreads) void k_concat(CatArgs a, float* __restrict__ cat,
                                                     const float* __restrict__ gcat, int64_t N,
                                                     int64_t HW) {
    using T = typename std::conditional<V == 4, float4, float>::type;
    const int64_t C_total = a.c_off[a.K];
    for (int64_t q = blockIdx.y; q < N * a.K; q += gridDim.y) {
        const int k = (int)(q % a.K);
        const int64_t n = q / a.K;
        const int64_t Ck = a.c_off[k + 1] - a.c_off[k];
        const int64_t len = Ck * HW / V;
        const int64_t coff = (n * C_total + a.c_off[k]) * HW / V, poff = n * Ck * HW / V;
        if (BWD) {
            T* d = reinterpret_cast<T*>(a.piece[k]);
            if (!d) continue;
            d += poff;
            const T* src = reinterpret_cast<const T*>(gcat) + coff;
            const bool acc = (a.acc_mask >> k) & 1;
            for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < len;
                 i += (int64_t)gridDim.x * kThreads) {
                T v = src[i];
                if (acc) {
                    const T o = d[i];
                    if constexpr (V == 4) {
                        v.x += o.x;
                        v.y += o.y;
                        v.z += o.z;
                        v.w += o.w;
                    } else {
                        v += o;
                    }
                }
                d[i] = v;
            }
        } else {
            const T* src = reinterpret_cast<const T*>(a.piece[k]) + poff;
            T* d = reinterpret_cast<T*>(cat) + coff;
            for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < len;
                 i += (int64_t)gridDim.x * kThreads)
                d[i] = src[i];
        }
    }
}

// ---------------------------------------------------------------------------
// Multi-tensor operators.  The tensors are cut into chunks of kMtChunk
// elements; every block first builds, in LDS, the prefix count of chunks
// per tensor from the size table, then walks chunks blockIdx.x,
// blockIdx.x + gridDim.x, ... and finds each chunk's tensor by binary
// search.  Work is balanced over blocks whatever the tensor sizes, and no
// block reads more of the table than the prologue does.
// ---------------------------------------------------------------------------
constexpr int kMultiBlocks = 512;
constexpr int64_t kMtChunk = 4096;

struct ChunkMap {
    int* pref;  // LDS: pref[k] = chunks before tensor k, pref[n] = total
    int n;
    __device__ int total() const { return pref[n]; }
    // tensor holding chunk c, and the chunk's first element in it
    __device__ void locate(int c, int* k, int64_t* first) const {
        int lo = 0, hi = n;  // pref[lo] <= c < pref[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (pref[mid] <= c)
                lo = mid;
            else
                hi = mid;
        }
        *k = lo;
        *first = (int64_t)(c - pref[lo]) * kMtChunk;
    }
};

// Builds the chunk prefix of `numel` (n <= kMaxMultiTensors) in `pref`.
__device__ ChunkMap build_chunk_map(const int64_t* __restrict__ numel, int n, int* pref) {
    const int t = threadIdx.x;
    constexpr int kSeg = (kMaxMultiTensors + kThreads - 1) / kThreads;
    // each thread counts a contiguous segment, then a scan over the 256
    // segment totals gives each segment's offset
    __shared__ int seg[kThreads];
    int local[kSeg];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
        const int k = t * kSeg + i;
        const int c = k < n ? (int)((numel[k] + kMtChunk - 1) / kMtChunk) : 0;
        local[i] = c;
        sum += c;
    }
    seg[t] = sum;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {  // inclusive Hillis-Steele scan
        const int v = t >= off ? seg[t - off] : 0;
        __syncthreads();
        seg[t] += v;
        __syncthreads();
    }
    int run = seg[t] - sum;  // exclusive prefix of this segment
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
        const int k = t * kSeg + i;
        if (k < n) pref[k] = run;
        run += local[i];
    }
    if (t == kThreads - 1) pref[n] = seg[kThreads - 1];
    __syncthreads();
    return ChunkMap{pref, n};
}

__global__ __launch_bounds__(kThreads) void k_multi_norm_sq(const float* const* __restrict__ t,
                                                            const int64_t* __restrict__ numel,
                                                            int n_tensors,
                                                            double* __restrict__ part) {
    __shared__ int pref[kMaxMultiTensors + 1];
    __shared__ double sh[kThreads];
    const ChunkMap map = build_chunk_map(numel, n_tensors, pref);
    double s = 0.0;
    for (int c = blockIdx.x; c < map.total(); c += gridDim.x) {
        int k;
        int64_t first;
        map.locate(c, &k, &first);
        const float* p = t[k];
        const int64_t end = min(first + kMtChunk, numel[k]);
        for (int64_t i = first + threadIdx.x; i < end; i += kThreads) {
            const double v = p[i];
            s += v * v;
        }
    }
    s = block_sum(s, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ __launch_bounds__(kThreads) void k_multi_norm_finish(const double* __restrict__ part,
                                                                int nparts,
                                                                double* __restrict__ out) {
    __shared__ double sh[kThreads];
    double s = 0.0;
    for (int b = threadIdx.x; b < nparts; b += kThreads) s += part[b];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) out[0] = s;
}

// t[k][i] = value (FILL) or t[k][i] *= value
template <bool FILL>
__global__ __launch_bounds__(kThreads) void k_multi_set(float* const* __restrict__ t,
                                                        const int64_t* __restrict__ numel,
                                                        int n_tensors, float value) {
    __shared__ int pref[kMaxMultiTensors + 1];
    const ChunkMap map = build_chunk_map(numel, n_tensors, pref);
    for (int c = blockIdx.x; c < map.total(); c += gridDim.x) {
        int k;
        int64_t first;
        map.locate(c, &k, &first);
        float* p = t[k];
        const int64_t end = min(first + kMtChunk, numel[k]);
        for (int64_t i = first + threadIdx.x; i < end; i += kThreads) p[i] = FILL ? value : p[i] * value;
    }
}

// Gradient clip with the coefficient formed on the device from the squared
// norm (norm_sq[0], float64), as the host does it: total = (float)sqrt(sq);
// when total > max_norm and total > 1e-6 every tensor is scaled by
// max_norm / total (one fp32 division), else nothing changes.
__global__ __launch_bounds__(kThreads) void k_multi_clip(float* const* __restrict__ t,
                                                         const int64_t* __restrict__ numel,
                                                         int n_tensors,
                                                         const double* __restrict__ norm_sq,
                                                         float max_norm) {
#pragma clang fp contract(off)
    const float total = (float)sqrt(norm_sq[0]);
    if (!(total > max_norm && total > 1e-6f)) return;  // uniform over the grid
    const float coef = max_norm / total;
    __shared__ int pref[kMaxMultiTensors + 1];
    const ChunkMap map = build_chunk_map(numel, n_tensors, pref);
    for (int c = blockIdx.x; c < map.total(); c += gridDim.x) {
        int k;
        int64_t first;
        map.locate(c, &k, &first);
        float* p = t[k];
        const int64_t end = min(first + kMtChunk, numel[k]);
        for (int64_t i = first + threadIdx.x; i < end; i += kThreads) p[i] = p[i] * coef;
    }
}

// The AdamW update of adamw.cpp:60-108, operation by operation in fp32
// with no fused multiply-adds, so it matches a scalar IEEE evaluation of
// the same expressions bit for bit.
// scalars (device, optional): lr, step_size, sqrt_bc2 are read there
// instead of the arguments (a captured step replays with new values).
__global__ __launch_bounds__(kThreads) void k_adamw_multi(
    float* const* __restrict__ P, const float* const* __restrict__ G, float* const* __restrict__ M,
    float* const* __restrict__ V, const int64_t* __restrict__ numel, int n_tensors, float lr,
    float beta1, float beta2, float eps, float wd, float step_size, float sqrt_bc2,
    const float* __restrict__ scalars) {
#pragma clang fp contract(off)
    if (scalars) {
        lr = scalars[0];
        step_size = scalars[1];
        sqrt_bc2 = scalars[2];
    }
    __shared__ int pref[kMaxMultiTensors + 1];
    const ChunkMap map = build_chunk_map(numel, n_tensors, pref);
    const float one_m_b1 = 1.0f - beta1, one_m_b2 = 1.0f - beta2;
    const float lr_wd = lr * wd;
    for (int c = blockIdx.x; c < map.total(); c += gridDim.x) {
        int k;
        int64_t first;
        map.locate(c, &k, &first);
        float* theta = P[k];
        const float* g = G[k];
        float* m = M[k];
        float* v = V[k];
        const int64_t end = min(first + kMtChunk, numel[k]);
        for (int64_t i = first + threadIdx.x; i < end; i += kThreads) {
            const float gv = g[i];
            float th = theta[i];
            if (wd != 0.0f) th = th - lr_wd * th;
            const float mv = beta1 * m[i] + one_m_b1 * gv;
            const float vv = beta2 * v[i] + one_m_b2 * gv * gv;
            const float denom = (sqrtf(vv) / sqrt_bc2) + eps;
            th = th - step_size * (mv / denom);
            m[i] = mv;
            v[i] = vv;
            theta[i] = th;
        }
    }
}

// The device training step's tail in one launch: the gradient norm's
// finish (k_multi_norm_finish's sum of the block partials, formed by every
// block in the same order; block 0 writes it to norm_out), the clip
// (k_multi_clip's decision, the clipped gradient kept in a register), the
// AdamW update (k_adamw_multi) and, with zero_grad, the gradients set to
// zero (k_multi_set, Module::zero_grad after the step): the values of those
// four launches.
__global__ __launch_bounds__(kThreads) void k_adamw_clip_multi(
    float* const* __restrict__ P, float* const* __restrict__ G, float* const* __restrict__ M,
    float* const* __restrict__ V, const int64_t* __restrict__ numel, int n_tensors, float beta1,
    float beta2, float eps, float wd, const float* __restrict__ scalars,
    const double* __restrict__ part, int nparts, double* __restrict__ norm_out, float max_norm,
    int zero_grad) {
#pragma clang fp contract(off)
    __shared__ double sh[kThreads];
    __shared__ double sq_all;
    double s = 0.0;
    for (int b = threadIdx.x; b < nparts; b += kThreads) s += part[b];
    s = block_sum(s, sh);
    if (threadIdx.x == 0) {
        sq_all = s;
        if (blockIdx.x == 0) norm_out[0] = s;
    }
    __syncthreads();
    const float total = (float)sqrt(sq_all);
    const bool clip = total > max_norm && total > 1e-6f;  // uniform over the grid
    const float coef = clip ? max_norm / total : 1.0f;
    const float lr = scalars[0], step_size = scalars[1], sqrt_bc2 = scalars[2];
    __shared__ int pref[kMaxMultiTensors + 1];
    const ChunkMap map = build_chunk_map(numel, n_tensors, pref);
    const float one_m_b1 = 1.0f - beta1, one_m_b2 = 1.0f - beta2;
    const float lr_wd = lr * wd;
    for (int c = blockIdx.x; c < map.total(); c += gridDim.x) {
        int k;
        int64_t first;
        map.locate(c, &k, &first);
        float* theta = P[k];
        float* g = G[k];
        float* m = M[k];
        float* v = V[k];
        const int64_t end = min(first + kMtChunk, numel[k]);
        for (int64_t i = first + threadIdx.x; i < end; i += kThreads) {
            float gv = g[i];
            if (clip) gv = gv * coef;
            float th = theta[i];
            if (wd != 0.0f) th = th - lr_wd * th;
            const float mv = beta1 * m[i] + one_m_b1 * gv;
            const float vv = beta2 * v[i] + one_m_b2 * gv * gv;
            const float denom = (sqrtf(vv) / sqrt_bc2) + eps;
            th = th - step_size * (mv / denom);
            m[i] = mv;
            v[i] = vv;
            theta[i] = th;
            g[i] = zero_grad ? 0.0f : gv;
        }
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
hipError_t launch_conv_forward(const float* in, const float* w, const float* bias, float* out,
                               const ConvShape& c, hipStream_t s) {
    const int64_t total = c.N * c.C_out * c.Ho * c.Wo;
    if (conv_dense_small(c)) {
        // all of C_out per thread up to 16 channels, else tiles of 16 / 8 / 4
        const int64_t pos = c.N * c.Ho * c.Wo;
        const int ct = c.C_out % 16 == 0 ? 16 : c.C_out % 8 == 0 ? 8 : 4;
        const dim3 grid((unsigned)((pos + kThreads - 1) / kThreads), (unsigned)(c.C_out / ct));
        if (ct == 16)
            k_conv_fwd_co<16><<<grid, kThreads, 0, s>>>(in, w, bias, out, c);
        else if (ct == 8)
            k_conv_fwd_co<8><<<grid, kThreads, 0, s>>>(in, w, bias, out, c);
        else
            k_conv_fwd_co<4><<<grid, kThreads, 0, s>>>(in, w, bias, out, c);
        return hipGetLastError();
    }
    k_conv_fwd<<<blocks_for(total), kThreads, 0, s>>>(in, w, bias, out, c);
    return hipGetLastError();
}

size_t conv_backward_workspace_bytes(const ConvShape& c) {
    const int64_t rows = c.C_out * (c.C_in / c.groups) * (c.K * c.K + 1);
    return (size_t)(rows * conv_dw_chunks(c)) * sizeof(double);
}

hipError_t launch_conv_backward(const float* go, const float* in, const float* w, float* gx,
                                float* gw, float* gb, const ConvShape& c, bool accumulate_dx,
                                void* ws, hipStream_t s) {
    if (gx) {
        const int64_t total = c.N * c.C_in * c.H * c.W;
        if (accumulate_dx)
            k_conv_dx<true><<<blocks_for(total), kThreads, 0, s>>>(go, w, gx, c);
        else
            k_conv_dx<false><<<blocks_for(total), kThreads, 0, s>>>(go, w, gx, c);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if ((gw || gb) && conv_dw_dense(c)) {
        const int64_t csize = conv_dense_chunk(c), chunks = conv_dw_chunks(c);
        double* part = static_cast<double*>(ws);
        const int64_t waves = (c.C_out / kConvCoW) * c.C_in;
        const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)chunks);
        if (c.K == 3)
            k_conv_dw_co<3><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize);
        else
            k_conv_dw_co<1><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t rows = c.C_out * c.C_in * (c.K * c.K + 1);
        k_conv_dw_finish_wave<<<(unsigned)((rows + 3) / 4), kThreads, 0, s>>>(part, gw, gb, c,
                                                                             chunks);
        return hipGetLastError();
    }
    if (gw || gb) {
        const int64_t chunks = conv_chunks(c), csize = conv_chunk(c);
        const int64_t cig = c.C_in / c.groups;
        double* part = static_cast<double*>(ws);
        const bool taps = (c.K == 1 || c.K == 3 || c.K == 5 || c.K == 7) &&
                          c.N * c.Ho * c.Wo < ((int64_t)1 << 31) && c.H < ((int64_t)1 << 30) &&
                          c.W < ((int64_t)1 << 30);
        if (taps) {
            const dim3 grid((unsigned)(c.C_out * cig), (unsigned)chunks);
            switch (c.K) {
                case 1: k_conv_dw_taps<1><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize); break;
                case 3: k_conv_dw_taps<3><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize); break;
                case 5: k_conv_dw_taps<5><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize); break;
                default: k_conv_dw_taps<7><<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize); break;
            }
        } else {
            dim3 grid((unsigned)(c.C_out * cig * (c.K * c.K + 1)), (unsigned)chunks);
            k_conv_dw<<<grid, kThreads, 0, s>>>(go, in, part, c, chunks, csize);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const int64_t rows = c.C_out * cig * (c.K * c.K + 1);
        k_conv_dw_finish<<<blocks_for(rows), kThreads, 0, s>>>(part, gw, gb, c, chunks);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_sigmoid_forward(const float* x, float* y, int64_t n, hipStream_t s) {
    k_sigmoid_fwd<<<blocks_for(n), kThreads, 0, s>>>(x, y, n);
    return hipGetLastError();
}

hipError_t launch_sigmoid_backward(const float* gy, const float* y, float* gx, int64_t n,
                                   bool acc, hipStream_t s) {
    bsel(acc,
         [&](auto A) { k_sigmoid_bwd<A()><<<blocks_for(n), kThreads, 0, s>>>(gy, y, gx, n); });
    return hipGetLastError();
}

hipError_t launch_mul_broadcast_forward(const float* a, const float* b, float* y, int64_t rows,
                                        int64_t HW, hipStream_t s) {
    k_mul_bcast_fwd<<<blocks_for(rows * HW), kThreads, 0, s>>>(a, b, y, rows, HW);
    return hipGetLastError();
}

hipError_t launch_mul_broadcast_backward(const float* gy, const float* a, const float* b,
                                         float* ga, float* gb, int64_t rows, int64_t HW, bool acc,
                                         hipStream_t s) {
    bsel(acc, [&](auto A) {
        k_mul_bcast_bwd<A()><<<(unsigned)rows, kThreads, 0, s>>>(gy, a, b, ga, gb, HW);
    });
    return hipGetLastError();
}

hipError_t launch_convex_forward(const float* g, const float* a, const float* b, float* y,
                                 int64_t n, hipStream_t s) {
    k_convex_fwd<<<blocks_for(n), kThreads, 0, s>>>(g, a, b, y, n);
    return hipGetLastError();
}

hipError_t launch_convex_backward(const float* gy, const float* g, const float* a,
                                  const float* b, float* gg, float* ga, float* gb, int64_t n,
                                  bool acc, hipStream_t s) {
    bsel(acc, [&](auto A) {
        k_convex_bwd<A()><<<blocks_for(n), kThreads, 0, s>>>(gy, g, a, b, gg, ga, gb, n);
    });
    return hipGetLastError();
}

hipError_t launch_sigmoid_convex_forward(const float* z, const float* a, const float* b,
                                         float* y, int64_t n, hipStream_t s) {
    k_sigmoid_convex_fwd<<<blocks_for(n), kThreads, 0, s>>>(z, a, b, y, n);
    return hipGetLastError();
}

hipError_t launch_sigmoid_convex_backward(const float* gy, const float* z, const float* a,
                                          const float* b, float* gz, float* ga, float* gb,
                                          int64_t n, bool acc, hipStream_t s) {
    bsel(acc, [&](auto A) {
        k_sigmoid_convex_bwd<A()><<<blocks_for(n), kThreads, 0, s>>>(gy, z, a, b, gz, ga, gb, n);
    });
    return hipGetLastError();
}

hipError_t launch_mul_sigmoid_forward(const float* a, const float* z, float* y, int64_t rows,
                                      int64_t HW, hipStream_t s) {
    k_mul_sigmoid_fwd<<<blocks_for(rows * HW), kThreads, 0, s>>>(a, z, y, rows, HW);
    return hipGetLastError();
}

hipError_t launch_mul_sigmoid_backward(const float* gy, const float* a, const float* z,
                                       float* ga, float* gz, int64_t rows, int64_t HW, bool acc,
                                       hipStream_t s) {
    bsel(acc, [&](auto A) {
        k_mul_sigmoid_bwd<A()><<<(unsigned)rows, kThreads, 0, s>>>(gy, a, z, ga, gz, HW);
    });
    return hipGetLastError();
}

hipError_t launch_avg_pool_forward(const float* in, float* out, int64_t rows, int64_t HW,
                                   hipStream_t s) {
    k_avg_pool_fwd<<<(unsigned)rows, kThreads, 0, s>>>(in, out, HW);
    return hipGetLastError();
}

hipError_t launch_avg_pool_backward(const float* go, float* gi, int64_t rows, int64_t HW,
                                    bool acc, hipStream_t s) {
    bsel(acc, [&](auto A) {
        k_avg_pool_bwd<A()><<<blocks_for(rows * HW), kThreads, 0, s>>>(go, gi, rows, HW);
    });
    return hipGetLastError();
}

hipError_t launch_upsample_forward(const float* in, float* out, int64_t rows, int64_t H_in,
                                   int64_t W_in, int64_t H_out, int64_t W_out, hipStream_t s) {
    if (std::max({H_in, W_in, H_out, W_out}) > INT32_MAX) return hipErrorInvalidValue;
    const float sh = (float)H_in / (float)H_out, sw = (float)W_in / (float)W_out;
    const dim3 grid = blocks_for(rows * H_out * W_out);
    auto run = [&](auto I) {
        using T = decltype(I);
        k_upsample_fwd<T><<<grid, kThreads, 0, s>>>(in, out, (T)rows, (T)H_in, (T)W_in,
                                                    (T)H_out, (T)W_out, sh, sw);
    };
    if (rows * std::max(H_in * W_in, H_out * W_out) <= INT32_MAX)
        run(int{});
    else
        run(int64_t{});
    return hipGetLastError();
}

hipError_t launch_upsample_backward(const float* go, float* gi, int64_t rows, int64_t H_in,
                                    int64_t W_in, int64_t H_out, int64_t W_out, bool acc,
                                    hipStream_t s) {
    if (std::max({H_in, W_in, H_out, W_out}) > INT32_MAX) return hipErrorInvalidValue;
    const float sh = (float)H_in / (float)H_out, sw = (float)W_in / (float)W_out;
    using std::integral_constant;
    // Tiles: the window of a TY x 64 tile spans at most (TY + 1) f + 6 rows
    // and 65 f + 6 columns at a factor f = out / in per axis; a column run
    // holds at most about 2.5 f + 3 destinations.
    auto tiled = [&](auto TY, auto WR, auto WC, auto R) {
        const int64_t tiles_y = (H_in + TY() - 1) / TY(), tiles_x = (W_in + 63) / 64;
        const int64_t nt = rows * tiles_y * tiles_x;
        const unsigned grid = (unsigned)std::min<int64_t>(nt, (int64_t)1 << 20);
        bsel(acc, [&](auto A) {
            k_upsample_bwd_tiled<TY(), WR(), WC(), R(), A()><<<grid, kThreads, 0, s>>>(
                go, gi, rows, (int)H_in, (int)W_in, (int)H_out, (int)W_out, sh, sw,
                (int)tiles_y, (int)tiles_x);
        });
    };
    const bool i32 = rows * std::max(H_in * W_in, H_out * W_out) <= INT32_MAX;
    const int64_t f = H_out / H_in;
    if ((f == 2 || f == 4) && H_out == f * H_in && W_out == f * W_in &&
        std::max(H_out, W_out) <= ((int64_t)1 << 22)) {
        const dim3 grid = blocks_for(rows * H_in * W_in);
        auto run = [&](auto F, auto I) {
            using T = decltype(I);
            bsel(acc, [&](auto A) {
                k_upsample_bwd_int<F(), T, A()><<<grid, kThreads, 0, s>>>(go, gi, (T)rows,
                                                                          (int)H_in, (int)W_in,
                                                                          sh, sw);
            });
        };
        auto pick = [&](auto I) {
            if (f == 2)
                run(integral_constant<int, 2>{}, I);
            else
                run(integral_constant<int, 4>{}, I);
        };
        if (i32)
            pick(int{});
        else
            pick(int64_t{});
    } else if (H_out <= 2 * H_in && W_out <= 2 * W_in) {
        tiled(integral_constant<int, 8>{}, integral_constant<int, 24>{},
              integral_constant<int, 136>{}, integral_constant<int, 6>{});
    } else if (H_out <= 4 * H_in && W_out <= 4 * W_in) {
        tiled(integral_constant<int, 4>{}, integral_constant<int, 26>{},
              integral_constant<int, 266>{}, integral_constant<int, 10>{});
    } else {
        // larger factors: one thread per source pixel
        const dim3 grid = blocks_for(rows * H_in * W_in);
        auto run = [&](auto I) {
            using T = decltype(I);
            bsel(acc, [&](auto A) {
                k_upsample_bwd<10, T, A()><<<grid, kThreads, 0, s>>>(
                    go, gi, (T)rows, (int)H_in, (int)W_in, (int)H_out, (int)W_out, sh, sw);
            });
        };
        if (i32)
            run(int{});
        else
            run(int64_t{});
    }
    return hipGetLastError();
}

hipError_t launch_pixel_shuffle(const float* in, float* out, int64_t N, int64_t C_in,
                                int64_t H_in, int64_t W_in, int64_t r, bool backward, bool acc,
                                hipStream_t s) {
    const int64_t C_out = C_in / (r * r);
    const int64_t total = N * C_out * H_in * r * W_in * r;
    if (backward)
        bsel(acc, [&](auto A) {
            k_pixel_shuffle<true, A()><<<blocks_for(total), kThreads, 0, s>>>(in, out, N, C_out,
                                                                               H_in, W_in, r);
        });
    else
        k_pixel_shuffle<false, false><<<blocks_for(total), kThreads, 0, s>>>(in, out, N, C_out,
                                                                              H_in, W_in, r);
    return hipGetLastError();
}

hipError_t launch_pad_forward(const float* in, float* out, int64_t rows, int64_t H, int64_t W,
                              int64_t ph, int64_t pw, bool reflect, hipStream_t s) {
    const int64_t Hp = H + ph, Wp = W + pw;
    k_pad_fwd<<<blocks_for(rows * Hp * Wp), kThreads, 0, s>>>(in, out, rows, H, W, Hp, Wp,
                                                                reflect);
    return hipGetLastError();
}

hipError_t launch_pad_backward(const float* go, float* gi, int64_t rows, int64_t H, int64_t W,
                               int64_t ph, int64_t pw, bool reflect, hipStream_t s) {
    const int64_t Hp = H + ph, Wp = W + pw;
    k_pad_bwd<<<blocks_for(rows * H * W), kThreads, 0, s>>>(go, gi, rows, H, W, Hp, Wp,
                                                             reflect);
    return hipGetLastError();
}

hipError_t launch_crop(const float* in, float* out, int64_t rows, int64_t Hp, int64_t Wp,
                       int64_t H, int64_t W, bool backward, hipStream_t s) {
    if (backward)
        k_crop<true><<<blocks_for(rows * Hp * Wp), kThreads, 0, s>>>(in, out, rows, Hp, Wp, H,
                                                                      W);
    else
        k_crop<false><<<blocks_for(rows * H * W), kThreads, 0, s>>>(in, out, rows, Hp, Wp, H,
                                                                     W);
    return hipGetLastError();
}

size_t loss_sums_workspace_bytes(int64_t n) {
    return (size_t)(4 * blocks_for(n, kThreads, kLossBlocks) + 4) * sizeof(double);
}

hipError_t launch_loss_sums(const float* z, const float* y, int64_t n, float pos_weight,
                            double* out, void* ws, hipStream_t s) {
    const int nb = blocks_for(n, kThreads, kLossBlocks);
    double* part = static_cast<double*>(ws);
    k_loss_sums<<<nb, kThreads, 0, s>>>(z, y, n, pos_weight, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_loss_finish<<<1, kThreads, 0, s>>>(part, nb, out);
    return hipGetLastError();
}

hipError_t launch_dice_bce_backward(const float* z, const float* y, float* gz, int64_t n,
                                    float go, float w, float bw, float dw, float pos_weight,
                                    float smooth, float inter, float sum_p, float sum_y, bool acc,
                                    hipStream_t s, const double* sums) {
    const float scale_bce = bw > 0.0f ? (go * w * bw) / (float)n : 0.0f;
    const float scale_dice = dw > 0.0f ? go * w * dw : 0.0f;
    const float denom = sum_p + sum_y + smooth;
    const float numer = 2.0f * inter + smooth;
    bsel(acc, [&](auto A) {
        k_dice_bce_bwd<A()><<<blocks_for(n), kThreads, 0, s>>>(z, y, gz, n, scale_bce,
                                                               scale_dice, pos_weight, denom,
                                                               numer, smooth, sums);
    });
    return hipGetLastError();
}

hipError_t launch_sigmoid_threshold(const float* z, float* p, uint8_t* mask, int64_t n,
                                    float threshold, hipStream_t s) {
    k_sigmoid_threshold<<<blocks_for(n), kThreads, 0, s>>>(z, p, mask, n, threshold);
    return hipGetLastError();
}

hipError_t launch_concat(const CatArgs& a, float* cat, const float* gcat, int64_t N,
                         int64_t HW, bool backward, hipStream_t s) {
    int64_t max_len = 0;
    bool v4 = HW % 4 == 0 && ((uintptr_t)cat % 16 == 0) && ((uintptr_t)gcat % 16 == 0);
    for (int k = 0; k < a.K; ++k) {
        max_len = std::max(max_len, (a.c_off[k + 1] - a.c_off[k]) * HW);
        v4 = v4 && (uintptr_t)a.piece[k] % 16 == 0;
    }
    const int V = v4 ? 4 : 1;
    const int64_t bx = std::min<int64_t>((max_len / V + kThreads - 1) / kThreads, 1024);
    const dim3 grid((unsigned)std::max<int64_t>(bx, 1), (unsigned)std::min<int64_t>(N * a.K, 65535));
    auto run = [&](auto VV, auto B) {
        k_concat<VV(), B()><<<grid, kThreads, 0, s>>>(a, cat, gcat, N, HW);
    };
    bsel(backward, [&](auto B) {
        if (v4)
            run(std::integral_constant<int, 4>{}, B);
        else
            run(std::integral_constant<int, 1>{}, B);
    });
    return hipGetLastError();
}

size_t multi_norm_workspace_bytes() { return (size_t)(kMultiBlocks + 1) * sizeof(double); }

hipError_t launch_multi_norm_sq(const float* const* t, const int64_t* numel, int n_tensors,
                                double* out, void* ws, hipStream_t s) {
    double* part = static_cast<double*>(ws);
    k_multi_norm_sq<<<kMultiBlocks, kThreads, 0, s>>>(t, numel, n_tensors, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_multi_norm_finish<<<1, kThreads, 0, s>>>(part, kMultiBlocks, out);
    return hipGetLastError();
}

hipError_t launch_multi_scale(float* const* t, const int64_t* numel, int n_tensors, float scale,
                              hipStream_t s) {
    k_multi_set<false><<<kMultiBlocks, kThreads, 0, s>>>(t, numel, n_tensors, scale);
    return hipGetLastError();
}

hipError_t launch_multi_fill(float* const* t, const int64_t* numel, int n_tensors, float value,
                             hipStream_t s) {
    k_multi_set<true><<<kMultiBlocks, kThreads, 0, s>>>(t, numel, n_tensors, value);
    return hipGetLastError();
}

hipError_t launch_adamw_multi(float* const* p, const float* const* g, float* const* m,
                              float* const* v, const int64_t* numel, int n_tensors, float lr,
                              float beta1, float beta2, float eps, float wd, float step_size,
                              float sqrt_bc2, hipStream_t s, const float* scalars) {
    k_adamw_multi<<<kMultiBlocks, kThreads, 0, s>>>(p, g, m, v, numel, n_tensors, lr, beta1,
                                                     beta2, eps, wd, step_size, sqrt_bc2,
                                                     scalars);
    return hipGetLastError();
}

hipError_t launch_multi_norm_partials(const float* const* t, const int64_t* numel,
                                      int n_tensors, void* ws, hipStream_t s) {
    k_multi_norm_sq<<<kMultiBlocks, kThreads, 0, s>>>(t, numel, n_tensors,
                                                      static_cast<double*>(ws));
    return hipGetLastError();
}

hipError_t launch_adamw_clip_multi(float* const* p, float* const* g, float* const* m,
                                   float* const* v, const int64_t* numel, int n_tensors,
                                   float beta1, float beta2, float eps, float wd,
                                   const float* scalars, const void* norm_ws, double* norm_out,
                                   float max_norm, bool zero_grad, hipStream_t s) {
    k_adamw_clip_multi<<<kMultiBlocks, kThreads, 0, s>>>(
        p, g, m, v, numel, n_tensors, beta1, beta2, eps, wd, scalars,
        static_cast<const double*>(norm_ws), kMultiBlocks, norm_out, max_norm, zero_grad ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_multi_clip(float* const* t, const int64_t* numel, int n_tensors,
                             const double* norm_sq, float max_norm, hipStream_t s) {
    k_multi_clip<<<kMultiBlocks, kThreads, 0, s>>>(t, numel, n_tensors, norm_sq, max_norm);
    return hipGetLastError();
}

}  // namespace soar::ops
