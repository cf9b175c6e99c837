// wfinish.hip - deferred weight-gradient finishes.
//
// The convolution backward kernels leave their weight gradients as fp32
// partials per block, part[g][e] (g the block group, e the weight element),
// and a finish adds out[e] += sum_g part[g][e] in float64 with g ascending
// in 16 fixed segments (k_sum_partials for the pointwise weights and
// biases, k_dw_wgrad_finish for the depthwise taps and biases).  A model
// step runs one such finish per layer, 4-5 us of launch each for a few
// microseconds of work, and no weight gradient is read before the step's
// gradient clip (the reference's trainer clips, then steps the optimizer:
// src/engine/trainer.cpp:110-220).  With SOAR_DEFER_WEIGHT_FINISH a
// backward call queues its finishes on the calling thread instead, and
// soar_weight_grad_flush runs every queued finish in one launch: block b
// finds its table entry from the entries' first blocks and then does
// exactly what that entry's own finish would do, with the same segments in
// the same order, so the weight gradients are bit for bit those of the
// immediate finishes.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "gn_internal.hpp"

namespace soar {
namespace gn {
namespace {

// Entries of one launch: the table travels in the kernel arguments (by
// value, so a captured graph replays it as recorded).
constexpr int kFinishMax = 64;
// Entries of at most this many partials per element run one element per
// thread (1024 per block), the others one element per lane of each of 16
// waves (64 per block, a wave per segment).
constexpr int64_t kNarrowG = 32;
constexpr int kNarrowBatch = 16;  // loads a thread keeps in flight

struct FinishTable {
    int n;
    int64_t first[kFinishMax + 1];  // first block of entry i; first[n] = grid size
    const float* part[kFinishMax];
    float* out0[kFinishMax];
    float* out1[kFinishMax];
    int64_t E[kFinishMax];
    int64_t G[kFinishMax];
    int64_t kk1[kFinishMax];
};
static_assert(sizeof(FinishTable) < 4096, "kernel argument size");

// out0 / out1 element that entry i's element e adds into (null: none)
__device__ __forceinline__ float* finish_target(const FinishTable& t, int i, int64_t e) {
    const int64_t kk1 = t.kk1[i];
    if (kk1 == 0) return t.out0[i] + e;  // k_sum_partials: out0[e]
    // k_dw_wgrad_finish: taps c*(kk1-1) + k of out0, bias c of out1
    const int64_t c = e / kk1, k = e - c * kk1;
    return k < kk1 - 1 ? (t.out0[i] ? t.out0[i] + c * (kk1 - 1) + k : nullptr)
                       : (t.out1[i] ? t.out1[i] + c : nullptr);
}

// Every element's sum is the segment sums of segment_sum (segments
// [k*G/16, (k+1)*G/16), k = 0..15, each summed from 0.0 in g order) added
// in k order from 0.0, on either path.
__global__ __launch_bounds__(1024) void k_weight_finish(const FinishTable t) {
    __shared__ double lds[16][64];
    const int64_t b = blockIdx.x;
    // the entry whose blocks hold b (wave-uniform binary search)
    int lo = 0, hi = t.n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (t.first[mid] <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    const int i = lo;
    const float* __restrict__ part = t.part[i];
    const int64_t E = t.E[i], G = t.G[i];
    if (G <= kNarrowG) {
        // one element per thread: its G partials in batches of loads
        // issued together (rows clamped into range, the rest not added),
        // each segment's sum closed into the total as g passes its end
        const int64_t e = (b - t.first[i]) * 1024 + threadIdx.x;
        if (e >= E) return;
        double tsum = 0.0, sum = 0.0;
        int k = 0;
        int64_t end = G / 16;  // end of segment k
        for (int64_t g0 = 0; g0 < G; g0 += kNarrowBatch) {
            float v[kNarrowBatch];
#pragma unroll
            for (int u = 0; u < kNarrowBatch; ++u) v[u] = part[min(g0 + u, G - 1) * E + e];
#pragma unroll
            for (int u = 0; u < kNarrowBatch; ++u) {
                const int64_t g = g0 + u;
                if (g < G) {
                    while (g >= end) {
                        tsum += sum;
                        sum = 0.0;
                        ++k;
                        end = (k + 1) * G / 16;
                    }
                    sum += (double)v[u];
                }
            }
        }
        for (; k < 16; ++k) {
            tsum += sum;
            sum = 0.0;
        }
        float* o = finish_target(t, i, e);
        if (o) *o = (float)((double)*o + tsum);
        return;
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t e = (b - t.first[i]) * 64 + lane;
    const int64_t g0 = wv * G / 16, g1 = (wv + 1) * G / 16;
    const double sum = e < E ? segment_sum(part, E, e, g0, g1) : 0.0;
    lds[wv][lane] = sum;
    __syncthreads();
    if (wv == 0 && e < E) {
        double tsum = 0.0;
#pragma unroll
        for (int k = 0; k < 16; ++k) tsum += lds[k][lane];
        float* o = finish_target(t, i, e);
        if (o) *o = (float)((double)*o + tsum);
    }
}

struct Pending {
    std::vector<WeightFinish> list;
    hipStream_t stream = nullptr;
    bool defer = false;  // the current C-ABI call defers its finishes
};
thread_local Pending g_pending;

// the element range [p, p + n) an entry writes
bool overlaps(const float* a, int64_t na, const float* b, int64_t nb) {
    if (!a || !b) return false;
    return a < b + nb && b < a + na;
}

void out_ranges(const WeightFinish& f, const float** p0, int64_t* n0, const float** p1,
                int64_t* n1) {
    if (f.kk1 == 0) {
        *p0 = f.out0, *n0 = f.E, *p1 = nullptr, *n1 = 0;
    } else {
        const int64_t C = f.E / f.kk1;
        *p0 = f.out0, *n0 = C * (f.kk1 - 1), *p1 = f.out1, *n1 = C;
    }
}

bool clash(const WeightFinish& a, const WeightFinish& b) {
    const float *a0, *a1, *b0, *b1;
    int64_t na0, na1, nb0, nb1;
    out_ranges(a, &a0, &na0, &a1, &na1);
    out_ranges(b, &b0, &nb0, &b1, &nb1);
    return overlaps(a0, na0, b0, nb0) || overlaps(a0, na0, b1, nb1) ||
           overlaps(a1, na1, b0, nb0) || overlaps(a1, na1, b1, nb1);
}

}  // namespace

void weight_finish_defer(bool on) { g_pending.defer = on; }

bool weight_finish_deferring() { return g_pending.defer; }

hipError_t weight_finish_flush() {
    Pending& pd = g_pending;
    if (pd.list.empty()) return hipSuccess;
    const hipStream_t s = pd.stream;  // the partials' writers ran there
    size_t k = 0;
    while (k < pd.list.size()) {
        FinishTable t{};
        int64_t blocks = 0;
        while (k < pd.list.size() && t.n < kFinishMax) {
            const WeightFinish& f = pd.list[k++];
            const int i = t.n++;
            t.first[i] = blocks;
            t.part[i] = f.part;
            t.out0[i] = f.out0;
            t.out1[i] = f.out1;
            t.E[i] = f.E;
            t.G[i] = f.G;
            t.kk1[i] = f.kk1;
            blocks += f.G <= kNarrowG ? (f.E + 1023) / 1024 : (f.E + 63) / 64;
        }
        t.first[t.n] = blocks;
        const int tok = prof_begin(s, "weight_grad_finish");
        k_weight_finish<<<dim3((unsigned)blocks), 1024, 0, s>>>(t);
        prof_end(s, tok);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            pd.list.clear();
            return e;
        }
    }
    pd.list.clear();
    return hipSuccess;
}

bool weight_finish_queue(const WeightFinish& f, hipStream_t s, hipError_t* err) {
    Pending& pd = g_pending;
    *err = hipSuccess;
    if (!pd.defer || f.E <= 0) return false;
    // one stream per queue, and no two queued finishes add into the same
    // weights (their read-modify-writes would race): flush first
    bool flush = !pd.list.empty() && pd.stream != s;
    for (size_t i = 0; !flush && i < pd.list.size(); ++i) flush = clash(pd.list[i], f);
    if (flush && (*err = weight_finish_flush()) != hipSuccess) return true;
    pd.stream = s;
    pd.list.push_back(f);
    return true;
}

hipError_t weight_finish_before(const float* o0, int64_t n0, const float* o1, int64_t n1,
                                hipStream_t s, bool defer) {
    Pending& pd = g_pending;
    if (pd.list.empty()) return hipSuccess;
    bool flush = defer && pd.stream != s;
    for (size_t i = 0; !flush && i < pd.list.size(); ++i) {
        const float *a0, *a1;
        int64_t na0, na1;
        out_ranges(pd.list[i], &a0, &na0, &a1, &na1);
        flush = overlaps(a0, na0, o0, n0) || overlaps(a0, na0, o1, n1) ||
                overlaps(a1, na1, o0, n0) || overlaps(a1, na1, o1, n1);
    }
    return flush ? weight_finish_flush() : hipSuccess;
}

size_t weight_finish_pending() { return g_pending.list.size(); }

hipStream_t weight_finish_stream() { return g_pending.stream; }

void weight_finish_discard() { g_pending.list.clear(); }

}  // namespace gn
}  // namespace soar
