// elementwise.hip - the stand-alone elementwise operators of the path:
// SiLU forward/backward, residual add and its gradient merge, fill/zero.
//
// Reference kernels (pomagrenate/soar.cpp): src/cuda/ops/
// activation_kernels.cu:11-130 (SiLU), binary_ops_kernels.cu:12-102
// (zero, fill, add, add_backward), shaders/tensor_add.comp:21-28.
// All are one streaming pass; blocks walk the tensor with a grid stride in
// 128-bit steps when every pointer is 16-byte aligned, else element-wise.
#include "gn_internal.hpp"
#include "gn_math.hpp"

namespace soar {
namespace gn {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

struct SiluFwd {
    __device__ float operator()(float v) const { return v * sigmoid_fast(v); }
};

// Unary map y = op(x), 128-bit or scalar.
template <typename Op, bool VEC>
__global__ __launch_bounds__(256) void k_map(const float* __restrict__ x,
                                             float* __restrict__ y, int64_t n,
                                             Op op) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        const f4* x4 = reinterpret_cast<const f4*>(x);
        f4* y4 = reinterpret_cast<f4*>(y);
        const int64_t n4 = n >> 2;
        for (int64_t j = i; j < n4; j += stride) {
            f4 v = x4[j];
            f4 o = {op(v.x), op(v.y), op(v.z), op(v.w)};
            y4[j] = o;
        }
        for (int64_t j = n4 * 4 + i; j < n; j += stride) y[j] = op(x[j]);
    } else {
        for (int64_t j = i; j < n; j += stride) y[j] = op(x[j]);
    }
}

// grad_x += grad_y * s * (1 + x*(1-s))
template <bool VEC>
__global__ __launch_bounds__(256) void k_silu_bwd(const float* __restrict__ gy,
                                                  const float* __restrict__ x,
                                                  float* __restrict__ gx,
                                                  int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    auto f = [](float g, float v) {
        float s = sigmoid_fast(v);
        return g * s * fmaf(v, 1.0f - s, 1.0f);
    };
    int64_t done = 0;
    if (VEC) {
        const f4* g4 = reinterpret_cast<const f4*>(gy);
        const f4* x4 = reinterpret_cast<const f4*>(x);
        f4* o4 = reinterpret_cast<f4*>(gx);
        const int64_t n4 = n >> 2;
        for (int64_t j = i; j < n4; j += stride) {
            f4 g = g4[j], v = x4[j], o = o4[j];
            o.x += f(g.x, v.x);
            o.y += f(g.y, v.y);
            o.z += f(g.z, v.z);
            o.w += f(g.w, v.w);
            o4[j] = o;
        }
        done = n4 * 4;
    }
    for (int64_t j = done + i; j < n; j += stride) gx[j] += f(gy[j], x[j]);
}

template <bool VEC>
__global__ __launch_bounds__(256) void k_add(const float* __restrict__ a,
                                             const float* __restrict__ b,
                                             float* __restrict__ y, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t done = 0;
    if (VEC) {
        const f4* a4 = reinterpret_cast<const f4*>(a);
        const f4* b4 = reinterpret_cast<const f4*>(b);
        f4* y4 = reinterpret_cast<f4*>(y);
        const int64_t n4 = n >> 2;
        for (int64_t j = i; j < n4; j += stride) y4[j] = a4[j] + b4[j];
        done = n4 * 4;
    }
    for (int64_t j = done + i; j < n; j += stride) y[j] = a[j] + b[j];
}

// acc += g for one or two accumulators (either may be null).
template <bool VEC>
__global__ __launch_bounds__(256) void k_accumulate(const float* __restrict__ g,
                                                    float* __restrict__ ga,
                                                    float* __restrict__ gb,
                                                    int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t done = 0;
    if (VEC) {
        const f4* g4 = reinterpret_cast<const f4*>(g);
        f4* a4 = reinterpret_cast<f4*>(ga);
        f4* b4 = reinterpret_cast<f4*>(gb);
        const int64_t n4 = n >> 2;
        for (int64_t j = i; j < n4; j += stride) {
            f4 v = g4[j];
            if (ga) a4[j] += v;
            if (gb) b4[j] += v;
        }
        done = n4 * 4;
    }
    for (int64_t j = done + i; j < n; j += stride) {
        float v = g[j];
        if (ga) ga[j] += v;
        if (gb) gb[j] += v;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void k_fill(float* __restrict__ p, float v,
                                              int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t done = 0;
    if (VEC) {
        f4* p4 = reinterpret_cast<f4*>(p);
        const f4 w = {v, v, v, v};
        const int64_t n4 = n >> 2;
        for (int64_t j = i; j < n4; j += stride) p4[j] = w;
        done = n4 * 4;
    }
    for (int64_t j = done + i; j < n; j += stride) p[j] = v;
}

inline bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Enough 256-thread blocks to fill 256 CUs several times over; the grid
// stride covers the rest.
inline dim3 grid_for(int64_t n) {
    int64_t want = (n / 4 + 255) / 256;
    if (want < 1) want = 1;
    if (want > 16384) want = 16384;
    return dim3((unsigned)want);
}

}  // namespace

hipError_t launch_silu_forward(const float* x, float* y, int64_t n, hipStream_t s) {
    int tok = prof_begin(s, "silu_forward");
    if (aligned16(x) && aligned16(y))
        k_map<SiluFwd, true><<<grid_for(n), 256, 0, s>>>(x, y, n, SiluFwd{});
    else
        k_map<SiluFwd, false><<<grid_for(n), 256, 0, s>>>(x, y, n, SiluFwd{});
    prof_end(s, tok);
    return hipGetLastError();
}

hipError_t launch_silu_backward(const float* gy, const float* x, float* gx,
                                int64_t n, hipStream_t s) {
    int tok = prof_begin(s, "silu_backward");
    if (aligned16(gy) && aligned16(x) && aligned16(gx))
        k_silu_bwd<true><<<grid_for(n), 256, 0, s>>>(gy, x, gx, n);
    else
        k_silu_bwd<false><<<grid_for(n), 256, 0, s>>>(gy, x, gx, n);
    prof_end(s, tok);
    return hipGetLastError();
}

hipError_t launch_add_forward(const float* a, const float* b, float* y,
                              int64_t n, hipStream_t s) {
    int tok = prof_begin(s, "add_forward");
    if (aligned16(a) && aligned16(b) && aligned16(y))
        k_add<true><<<grid_for(n), 256, 0, s>>>(a, b, y, n);
    else
        k_add<false><<<grid_for(n), 256, 0, s>>>(a, b, y, n);
    prof_end(s, tok);
    return hipGetLastError();
}

hipError_t launch_add_backward(const float* gy, float* ga, float* gb, int64_t n,
                               hipStream_t s) {
    int tok = prof_begin(s, "add_backward");
    if (aligned16(gy) && aligned16(ga) && aligned16(gb))
        k_accumulate<true><<<grid_for(n), 256, 0, s>>>(gy, ga, gb, n);
    else
        k_accumulate<false><<<grid_for(n), 256, 0, s>>>(gy, ga, gb, n);
    prof_end(s, tok);
    return hipGetLastError();
}

hipError_t launch_fill(float* p, float v, int64_t n, hipStream_t s) {
    int tok = prof_begin(s, "fill");
    if (aligned16(p))
        k_fill<true><<<grid_for(n), 256, 0, s>>>(p, v, n);
    else
        k_fill<false><<<grid_for(n), 256, 0, s>>>(p, v, n);
    prof_end(s, tok);
    return hipGetLastError();
}

}  // namespace gn
}  // namespace soar
