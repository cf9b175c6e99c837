// capi.cpp - the C-ABI of libsoar_gn.so (declared in include/soar_gn.h).
//
// Responsibilities: argument validation (shapes, flags, and that every
// device pointer lies inside one device allocation large enough for the
// bytes the kernels will touch), status codes with a per-thread message,
// the library-owned workspace of the reference-signature entry points,
// the device arena, and optional per-kernel hipEvent timing.
//
// Error convention: the reference returns silently on empty input
// (normalization_kernels.cu:96,255) and aborts on CUDA failure
// (cuda_common.cuh:35-43); the C boundary of the reference maps exceptions
// to -1 (src/api/c_api.cpp:33-35).  Here empty input is SOAR_OK with no
// launch, and every failure is a negative status, never an abort.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "capi_common.hpp"
#include "gn_internal.hpp"
#include "soar_gn.h"

using soar::gn::Plan;
using soar::gn::Tuning;

namespace soar::capi {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return SOAR_OK;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(SOAR_EHIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int device_count() {
    static std::once_flag once;
    static int count = 0;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        count = n;
        (void)hipGetLastError();
    });
    return count;
}

int require_device() {
    if (device_count() <= 0) return fail(SOAR_ENODEV, "no HIP device is visible");
    void* p = nullptr;
    (void)noalloc_scratch(&p);  // set-up; a failure is reported by the noalloc entry point
    return SOAR_OK;
}

// `p` must be device memory with at least `bytes` bytes from p to the end
// of its allocation.  A host pointer or a too-short buffer is rejected here
// rather than faulting the GPU.
int check_dev(const void* p, size_t bytes, const char* name) {
    if (!p) return fail(SOAR_EINVAL, "%s is NULL", name);
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    hipError_t e = hipMemGetAddressRange(&base, &size, const_cast<void*>(p));
    if (e != hipSuccess || !base) {
        (void)hipGetLastError();
        return fail(SOAR_EINVAL, "%s (%p) is not device memory", name, p);
    }
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    const uintptr_t q = reinterpret_cast<uintptr_t>(p);
    if (q < b || q - b > size || size - (q - b) < bytes)
        return fail(SOAR_EINVAL,
                    "%s (%p) needs %zu bytes but its allocation holds %zu from there",
                    name, p, bytes, (size_t)(size - (q - b)));
    return SOAR_OK;
}

int check_dev_opt(const void* p, size_t bytes, const char* name) {
    return p ? check_dev(p, bytes, name) : SOAR_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- library-owned workspace of the reference-signature entry points ------
struct OwnedWs {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::vector<OwnedWs> g_ws;

int owned_workspace(size_t need, void** out, void* stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    OwnedWs& w = g_ws[dev];
    if (w.bytes < need) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs);
        if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return fail(SOAR_EINVAL,
                        "the library-owned workspace must grow to %zu bytes (hipMalloc), which "
                        "a stream capture forbids; make one call of this shape before the "
                        "capture",
                        need);
        if (w.ptr) {
            e = hipFree(w.ptr);  // waits for work still using the old buffer
            w.ptr = nullptr;
            w.bytes = 0;
            if (e != hipSuccess) return hip_fail(e, "hipFree(workspace)");
        }
        size_t grow = std::max(need, (size_t)1 << 20);
        e = hipMalloc(&w.ptr, grow);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            w.ptr = nullptr;
            return fail(SOAR_ENOMEM, "hipMalloc of %zu workspace bytes failed", grow);
        }
        w.bytes = grow;
    }
    *out = w.ptr;
    return SOAR_OK;
}


}  // namespace soar::capi

using namespace soar::capi;

namespace {

// ---- tuning ---------------------------------------------------------------
std::mutex g_tune_mu;
Tuning g_tune;

Tuning current_tuning() {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    return g_tune;
}

// ---- shape validation shared by the fused entry points ---------------------
int check_shape(int64_t N, int64_t C, int64_t HW, int64_t G, int64_t* elems) {
    if (N < 0 || C < 0 || HW < 0)
        return fail(SOAR_EINVAL, "negative dimension (N=%lld C=%lld HW=%lld)",
                    (long long)N, (long long)C, (long long)HW);
    if (G <= 0) return fail(SOAR_EINVAL, "num_groups must be positive (G=%lld)", (long long)G);
    if (C % G != 0)
        return fail(SOAR_EINVAL, "C=%lld is not divisible by num_groups=%lld",
                    (long long)C, (long long)G);
    int64_t nc = 0, e = 0;
    if (__builtin_mul_overflow(N, C, &nc) || __builtin_mul_overflow(nc, HW, &e) ||
        e > INT64_MAX / 4)
        return fail(SOAR_EINVAL, "N*C*HW overflows");
    *elems = e;
    return SOAR_OK;
}

int check_ws(const Plan& p, void* ws, size_t ws_bytes) {
    const size_t need = soar::gn::workspace_bytes(p);
    if (ws_bytes < need)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu this shape needs",
                    ws_bytes, need);
    return check_dev(ws, need, "workspace");
}

// ---- per-kernel hipEvent timing --------------------------------------------
struct ProfRec {
    const char* name;
    hipEvent_t start, stop;
};
std::atomic<bool> g_prof_on{false};
std::mutex g_prof_mu;
std::vector<ProfRec> g_prof;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

}  // namespace

namespace soar {
namespace gn {

int prof_begin(hipStream_t s, const char* kernel) {
    if (!g_prof_on.load(std::memory_order_relaxed) || soar::capi::g_quiet_call) return -1;
    // no timing events inside a graph being captured
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    if (cs != hipStreamCaptureStatusNone) return -1;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    ProfRec r{kernel, take_event(), take_event()};
    if (!r.start || !r.stop) return -1;
    if (hipEventRecord(r.start, s) != hipSuccess) {
        (void)hipGetLastError();
        g_event_pool.push_back(r.start);
        g_event_pool.push_back(r.stop);
        return -1;
    }
    g_prof.push_back(r);
    return (int)g_prof.size() - 1;
}

void prof_end(hipStream_t s, int token) {
    if (token < 0) return;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (token < (int)g_prof.size() && hipEventRecord(g_prof[token].stop, s) != hipSuccess)
        (void)hipGetLastError();
}

}  // namespace gn
}  // namespace soar

namespace {

int check_pw_shape(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t* in_elems,
                   int64_t* out_elems) {
    if (N < 0 || C_in < 0 || C_out < 0 || HW < 0)
        return fail(SOAR_EINVAL, "negative dimension (N=%lld C_in=%lld C_out=%lld HW=%lld)",
                    (long long)N, (long long)C_in, (long long)C_out, (long long)HW);
    int64_t a = 0, b = 0, c = 0, d = 0, wsz = 0;
    if (__builtin_mul_overflow(N, C_in, &a) || __builtin_mul_overflow(a, HW, &b) ||
        __builtin_mul_overflow(N, C_out, &c) || __builtin_mul_overflow(c, HW, &d) ||
        __builtin_mul_overflow(C_in, C_out, &wsz) || b > INT64_MAX / 4 || d > INT64_MAX / 4 ||
        wsz > INT64_MAX / 4)
        return fail(SOAR_EINVAL, "pointwise convolution shape overflows");
    // (the backward runs the same kernel with C_out as its reduction axis)
    if (!soar::gn::pw_offsets_fit(std::max(C_in, C_out), HW))
        return fail(SOAR_EINVAL,
                    "HW=%lld or C=%lld exceeds the pointwise kernel's 32-bit in-sample offsets",
                    (long long)HW, (long long)std::max(C_in, C_out));
    *in_elems = b;
    *out_elems = d;
    return SOAR_OK;
}

// Grid of the convolution: one wave per (sample, pixel chunk).
bool pw_grid_fits(int64_t N, int64_t HW, int64_t chunk) {
    const int64_t cpp = (HW + chunk - 1) / chunk;
    return N <= (int64_t)0x7fffffff / std::max<int64_t>(cpp, 1);
}

}  // namespace

namespace {

int check_dw_shape(const soar::gn::DwShape& sh, int64_t* in_elems, int64_t* out_elems) {
    if (sh.N < 0 || sh.C < 0 || sh.Hi < 0 || sh.Wi < 0 || sh.Ho < 0 || sh.Wo < 0)
        return fail(SOAR_EINVAL, "negative dimension");
    if (sh.K <= 0 || sh.S <= 0 || sh.D <= 0 || sh.pad < 0)
        return fail(SOAR_EINVAL, "kernel size, stride and dilation must be positive, pad >= 0");
    int64_t nc = 0, a = 0, b = 0, c = 0, d = 0, kk = 0, span = 0;
    if (__builtin_mul_overflow(sh.N, sh.C, &nc) || __builtin_mul_overflow(nc, sh.Hi, &a) ||
        __builtin_mul_overflow(a, sh.Wi, &b) || __builtin_mul_overflow(nc, sh.Ho, &c) ||
        __builtin_mul_overflow(c, sh.Wo, &d) || __builtin_mul_overflow(sh.K, sh.K, &kk) ||
        __builtin_mul_overflow(sh.K - 1, sh.D, &span) || b > INT64_MAX / 4 ||
        d > INT64_MAX / 4 || kk > (1 << 20) || sh.pad > (1 << 30) || span > (1 << 30) ||
        sh.S > (1 << 20))
        return fail(SOAR_EINVAL, "depthwise convolution shape overflows");
    *in_elems = b;
    *out_elems = d;
    return SOAR_OK;
}

soar::gn::DwShape dw_shape(int64_t N, int64_t C, int64_t Hi, int64_t Wi, int64_t Ho,
                           int64_t Wo, int64_t K, int64_t pad, int64_t S, int64_t D) {
    soar::gn::DwShape sh;
    sh.N = N;
    sh.C = C;
    sh.Hi = Hi;
    sh.Wi = Wi;
    sh.Ho = Ho;
    sh.Wo = Wo;
    sh.K = K;
    sh.pad = pad;
    sh.S = S;
    sh.D = D;
    return sh;
}

bool dw_grids_fit(const soar::gn::DwShape& sh) {
    return soar::gn::dw_grid_blocks(sh, true) <= 0x7fffffff &&
           soar::gn::dw_grid_blocks(sh, false) <= 0x7fffffff;
}

}  // namespace

extern "C" {

SOAR_API const char* soar_last_error(void) { return g_err.c_str(); }

SOAR_API int soar_is_device_available(void) { return device_count() > 0 ? 1 : 0; }

SOAR_API size_t soar_gn_workspace_bytes(int64_t N, int64_t C, int64_t HW, int64_t G) {
    int64_t elems = 0;
    if (check_shape(N, C, HW, G, &elems) != SOAR_OK || elems == 0) return 0;
    Plan p;
    if (!soar::gn::make_plan(N, C, HW, G, current_tuning(), &p)) return 0;
    return soar::gn::workspace_bytes(p);
}

SOAR_API int soar_gn_silu_forward(const float* x, const float* gamma, const float* beta,
                                  float* y, float* mean, float* rstd, float* mean_lo,
                                  int64_t N, int64_t C, int64_t HW, int64_t G, float eps,
                                  unsigned flags, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    int64_t elems = 0;
    int rc = check_shape(N, C, HW, G, &elems);
    if (rc) return rc;
    if (flags & ~(SOAR_GN_SILU | SOAR_GN_RESIDUAL))
        return fail(SOAR_EINVAL, "unsupported forward flags 0x%x", flags);
    if (!(eps >= 0.0f)) return fail(SOAR_EINVAL, "eps must be >= 0");
    if (elems == 0) return ok();
    if ((rc = require_device())) return rc;
    const size_t tb = (size_t)elems * sizeof(float);
    const size_t sb = (size_t)(N * G) * sizeof(float);
    if ((rc = check_dev(x, tb, "x")) || (rc = check_dev(y, tb, "y")) ||
        (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
        (rc = check_dev_opt(mean_lo, sb, "mean_lo")) ||
        (rc = check_dev_opt(gamma, (size_t)C * 4, "gamma")) ||
        (rc = check_dev_opt(beta, (size_t)C * 4, "beta")))
        return rc;
    const Tuning t = current_tuning();
    Plan p;
    if (!soar::gn::make_plan(N, C, HW, G, t, &p))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    p.vec4 = p.vec4 && aligned16(x) && aligned16(y);
    if ((rc = check_ws(p, workspace, workspace_bytes))) return rc;
    soar::gn::FwdArgs a{x, gamma, beta, y, mean, rstd, mean_lo, eps, flags, workspace};
    hipError_t e = soar::gn::launch_forward(p, t, a, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "GroupNorm forward launch");
    return ok();
}

SOAR_API int soar_gn_silu_backward(const float* dy, const float* x, const float* gamma,
                                   const float* beta, const float* mean, const float* rstd,
                                   const float* mean_lo, float* dx, float* dgamma,
                                   float* dbeta, int64_t N,
                                   int64_t C, int64_t HW, int64_t G, unsigned flags,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    return soar::capi::gn_backward(dy, x, gamma, beta, mean, rstd, mean_lo, dx, dgamma, dbeta,
                                   N, C, HW, G, flags, workspace, workspace_bytes, stream,
                                   false);
}

}  // extern "C"

namespace soar::capi {

thread_local bool g_quiet_call = false;

DeferWeightFinish::DeferWeightFinish(bool on) : prev_(soar::gn::weight_finish_deferring()) {
    soar::gn::weight_finish_defer(prev_ || on);
}

DeferWeightFinish::~DeferWeightFinish() { soar::gn::weight_finish_defer(prev_); }

int weight_finish_room(const float* dweight, int64_t nw, const float* dbias, int64_t nb,
                       void* stream, unsigned flags) {
    const hipError_t e = soar::gn::weight_finish_before(
        dweight, dweight ? nw : 0, dbias, dbias ? nb : 0, static_cast<hipStream_t>(stream),
        (flags & SOAR_DEFER_WEIGHT_FINISH) != 0);
    return e == hipSuccess ? SOAR_OK : hip_fail(e, "weight-gradient finish launch");
}

int gn_backward(const float* dy, const float* x, const float* gamma, const float* beta,
                const float* mean, const float* rstd, const float* mean_lo, float* dx,
                float* dgamma, float* dbeta, int64_t N, int64_t C, int64_t HW, int64_t G,
                unsigned flags, void* workspace, size_t workspace_bytes, void* stream,
                bool ws_scratch) {
    int64_t elems = 0;
    int rc = check_shape(N, C, HW, G, &elems);
    if (rc) return rc;
    if (flags & ~(SOAR_GN_SILU | SOAR_GN_RESIDUAL | SOAR_GN_ACCUMULATE_DX))
        return fail(SOAR_EINVAL, "unsupported backward flags 0x%x", flags);
    if (elems == 0 || (!dx && !dgamma && !dbeta)) return ok();
    if ((rc = require_device())) return rc;
    const size_t tb = (size_t)elems * sizeof(float);
    const size_t sb = (size_t)(N * G) * sizeof(float);
    const size_t cb = (size_t)C * sizeof(float);
    if ((rc = check_dev(dy, tb, "dy")) || (rc = check_dev(x, tb, "x")) ||
        (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
        (rc = check_dev_opt(mean_lo, sb, "mean_lo")) || (rc = check_dev_opt(dx, tb, "dx")) || (rc = check_dev_opt(gamma, cb, "gamma")) ||
        (rc = check_dev_opt(beta, cb, "beta")) || (rc = check_dev_opt(dgamma, cb, "dgamma")) ||
        (rc = check_dev_opt(dbeta, cb, "dbeta")))
        return rc;
    const Tuning t = current_tuning();
    Plan p;
    if (!soar::gn::make_plan(N, C, HW, G, t, &p))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    p.vec4 = p.vec4 && aligned16(x) && aligned16(dy) && aligned16(dx);
    if (ws_scratch) {
        // the library's static scratch: its size is known, and it is not a
        // hipMalloc allocation to look up
        const size_t need = soar::gn::workspace_bytes(p);
        if (workspace_bytes < need)
            return fail(SOAR_EINVAL, "scratch of %zu bytes is smaller than the %zu this shape needs",
                        workspace_bytes, need);
    } else if ((rc = check_ws(p, workspace, workspace_bytes))) {
        return rc;
    }
    soar::gn::BwdArgs a{dy, x, gamma, beta, mean, rstd, mean_lo, dx, dgamma, dbeta, flags,
                        workspace};
    Tuning tl = t;
    if (ws_scratch) tl.streams = 1;  // the helper-stream pipeline would create a stream
    g_quiet_call = ws_scratch;       // and kernel timing would create events
    hipError_t e = soar::gn::launch_backward(p, tl, a, static_cast<hipStream_t>(stream));
    g_quiet_call = false;
    if (e != hipSuccess) return hip_fail(e, "GroupNorm backward launch");
    return ok();
}

}  // namespace soar::capi

extern "C" {

SOAR_API int soar_group_norm_forward(const float* in, const float* gamma, const float* beta,
                                     float* out, float* saved_mean, float* saved_rstd,
                                     size_t num_groups, size_t C, size_t HW, float eps,
                                     void* stream) {
    if (C == 0 || HW == 0) return ok();
    if (num_groups == 0 || C % num_groups)
        return fail(SOAR_EINVAL, "C=%zu is not divisible by num_groups=%zu", C, num_groups);
    int rc = require_device();
    if (rc) return rc;
    size_t need = soar_gn_workspace_bytes(1, (int64_t)C, (int64_t)HW, (int64_t)num_groups);
    if (need == 0) return fail(SOAR_EINVAL, "shape is too large");
    void* ws = nullptr;
    if ((rc = owned_workspace(need, &ws, stream))) return rc;
    return soar_gn_silu_forward(in, gamma, beta, out, saved_mean, saved_rstd, nullptr, 1,
                                (int64_t)C, (int64_t)HW, (int64_t)num_groups, eps, 0u, ws, need,
                                stream);
}

SOAR_API int soar_group_norm_backward(const float* grad_out, const float* in,
                                      const float* gamma, const float* saved_mean,
                                      const float* saved_rstd, float* grad_in,
                                      float* grad_gamma, float* grad_beta, size_t num_groups,
                                      size_t C, size_t HW, void* stream) {
    if (C == 0 || HW == 0) return ok();
    if (num_groups == 0 || C % num_groups)
        return fail(SOAR_EINVAL, "C=%zu is not divisible by num_groups=%zu", C, num_groups);
    int rc = require_device();
    if (rc) return rc;
    size_t need = soar_gn_workspace_bytes(1, (int64_t)C, (int64_t)HW, (int64_t)num_groups);
    if (need == 0) return fail(SOAR_EINVAL, "shape is too large");
    void* ws = nullptr;
    if ((rc = owned_workspace(need, &ws, stream))) return rc;
    return soar_gn_silu_backward(grad_out, in, gamma, nullptr, saved_mean, saved_rstd, nullptr,
                                 grad_in, grad_gamma, grad_beta, 1, (int64_t)C, (int64_t)HW,
                                 (int64_t)num_groups, SOAR_GN_ACCUMULATE_DX, ws, need, stream);
}

// ---- pointwise convolution --------------------------------------------------


SOAR_API int soar_conv2d_1x1_forward(const float* in, const float* weight, const float* bias,
                                     float* out, size_t C_in, size_t C_out, size_t HW,
                                     void* stream) {
    if (C_in > (size_t)INT64_MAX || C_out > (size_t)INT64_MAX || HW > (size_t)INT64_MAX)
        return fail(SOAR_EINVAL, "dimension too large");
    int64_t ie = 0, oe = 0;
    int rc = check_pw_shape(1, (int64_t)C_in, (int64_t)C_out, (int64_t)HW, &ie, &oe);
    if (rc) return rc;
    if (oe == 0) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    if ((rc = require_device())) return rc;
    if ((rc = check_dev(in, (size_t)ie * 4, "in")) ||
        (rc = check_dev(weight, C_in * C_out * 4, "weight")) ||
        (rc = check_dev_opt(bias, C_out * 4, "bias")) || (rc = check_dev(out, (size_t)oe * 4, "out")))
        return rc;
    const Tuning t = current_tuning();
    const int64_t chunk = soar::gn::pw_pick_chunk(1, (int64_t)C_out, (int64_t)HW, t.pw_chunk);
    if (!pw_grid_fits(1, (int64_t)HW, chunk))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    soar::gn::PwArgs a{in, weight, bias, out};
    hipError_t e = soar::gn::launch_pw_conv(a, 1, (int64_t)C_in, (int64_t)C_out, (int64_t)HW,
                                            chunk, nullptr, false, t.pw_small, nullptr, 1,
                                            static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "conv2d_1x1_forward launch");
}

SOAR_API int soar_pw_conv_forward(const float* x, const float* weight, const float* bias,
                                  float* z, int64_t N, int64_t C_in, int64_t C_out, int64_t HW,
                                  void* stream) {
    int64_t ie = 0, oe = 0;
    int rc = check_pw_shape(N, C_in, C_out, HW, &ie, &oe);
    if (rc) return rc;
    if (oe == 0) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    if ((rc = require_device())) return rc;
    if ((rc = check_dev(x, (size_t)ie * 4, "x")) ||
        (rc = check_dev(weight, (size_t)(C_in * C_out) * 4, "weight")) ||
        (rc = check_dev_opt(bias, (size_t)C_out * 4, "bias")) ||
        (rc = check_dev(z, (size_t)oe * 4, "z")))
        return rc;
    const Tuning t = current_tuning();
    const int64_t chunk = soar::gn::pw_pick_chunk(N, C_out, HW, t.pw_chunk);
    if (!pw_grid_fits(N, HW, chunk))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    soar::gn::PwArgs a{x, weight, bias, z};
    hipError_t e = soar::gn::launch_pw_conv(a, N, C_in, C_out, HW, chunk, nullptr, false,
                                            t.pw_small, nullptr, 1,
                                            static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "pointwise convolution launch");
}

// Offset of the split-K slices in the fused forward's workspace: after the
// GroupNorm's part, 256-byte aligned.
static size_t kz_offset(size_t gn_bytes) { return (gn_bytes + 255) & ~(size_t)255; }

SOAR_API size_t soar_pw_conv_gn_workspace_bytes(int64_t N, int64_t C_out, int64_t HW, int64_t G) {
    int64_t elems = 0;
    if (check_shape(N, C_out, HW, G, &elems) != SOAR_OK || elems == 0) return 0;
    const Tuning t = current_tuning();
    Plan p, q;
    if (!soar::gn::make_pw_plan(N, C_out, HW, G, t, &p)) return 0;
    size_t b = soar::gn::workspace_bytes(p);
    // small planes: a plain convolution, then the GroupNorm's own plan
    if (soar::gn::pw_use_small(N, C_out, 1, HW, t.pw_small) &&
        soar::gn::make_plan(N, C_out, HW, G, t, &q))
        b = std::max(b, soar::gn::workspace_bytes(q));
    // small grids: the split-K slices after the GroupNorm workspace
    const size_t kz = soar::gn::pw_kz_max_bytes(N, C_out, HW, p.chunk, (int)t.pw_kz);
    if (kz) b = std::max(b, kz_offset(soar::gn::workspace_bytes(p)) + kz);
    return b;
}

namespace {

// soar_pw_conv_gn_silu_forward, and with `residual` (non-null) its
// _add_forward form: y += residual in the apply pass (or, where the
// one-launch small-unit GroupNorm runs, in an add after it).
int pw_conv_gn_forward(const float* x, const float* weight, const float* bias,
                       const float* gamma, const float* beta, const float* residual, float* z,
                       float* y, float* mean, float* rstd, float* mean_lo, int64_t N,
                       int64_t C_in, int64_t C_out, int64_t HW, int64_t G, float eps,
                       unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
    int64_t ie = 0, oe = 0, elems = 0;
    int rc = check_pw_shape(N, C_in, C_out, HW, &ie, &oe);
    if (rc) return rc;
    if ((rc = check_shape(N, C_out, HW, G, &elems))) return rc;
    if (flags & ~SOAR_GN_SILU)
        return fail(SOAR_EINVAL, "unsupported flags 0x%x (SOAR_GN_SILU only)", flags);
    if (residual && (rc = check_dev(residual, (size_t)oe * 4, "residual"))) return rc;
    if (!(eps >= 0.0f)) return fail(SOAR_EINVAL, "eps must be >= 0");
    if (oe == 0) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    if ((rc = require_device())) return rc;
    const size_t sb = (size_t)(N * G) * sizeof(float);
    if ((rc = check_dev(x, (size_t)ie * 4, "x")) ||
        (rc = check_dev(weight, (size_t)(C_in * C_out) * 4, "weight")) ||
        (rc = check_dev_opt(bias, (size_t)C_out * 4, "bias")) ||
        (rc = check_dev_opt(gamma, (size_t)C_out * 4, "gamma")) ||
        (rc = check_dev_opt(beta, (size_t)C_out * 4, "beta")) ||
        (rc = check_dev(z, (size_t)oe * 4, "z")) || (rc = check_dev(y, (size_t)oe * 4, "y")) ||
        (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
        (rc = check_dev_opt(mean_lo, sb, "mean_lo")))
        return rc;
    const Tuning t = current_tuning();
    Plan p;
    if (!soar::gn::make_pw_plan(N, C_out, HW, G, t, &p) || !pw_grid_fits(N, HW, p.chunk))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    p.vec4 = p.vec4 && aligned16(z) && aligned16(y);
    if ((rc = check_ws(p, workspace, workspace_bytes))) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    soar::gn::PwArgs pa{x, weight, bias, z};
    Plan q;
    if (soar::gn::pw_use_small(N, C_out, C_in, HW, t.pw_small) &&
        soar::gn::make_plan(N, C_out, HW, G, t, &q)) {
        // Small planes: the SIMT convolution (no statistics epilogue), then
        // the GroupNorm forward over z with its own plan.
        q.vec4 = q.vec4 && aligned16(z) && aligned16(y) && (!residual || aligned16(residual));
        if ((rc = check_ws(q, workspace, workspace_bytes))) return rc;
        hipError_t e = soar::gn::launch_pw_conv(pa, N, C_in, C_out, HW, p.chunk, nullptr, false,
                                                t.pw_small, nullptr, 1, s);
        if (e != hipSuccess) return hip_fail(e, "pointwise convolution launch");
        soar::gn::FwdArgs a{z, gamma, beta, y, mean, rstd, mean_lo, eps, flags, workspace};
        const bool in_apply = residual && !soar::gn::forward_is_small(q, t);
        if (in_apply) {
            a.flags |= SOAR_GN_RESIDUAL;
            a.res = residual;
        }
        e = soar::gn::launch_forward(q, t, a, s);
        if (e != hipSuccess) return hip_fail(e, "GroupNorm forward launch");
        if (residual && !in_apply) {
            e = soar::gn::launch_add_forward(y, residual, y, oe, s);
            if (e != hipSuccess) return hip_fail(e, "residual add launch");
        }
        return ok();
    }
    // small grids split K over blocks when the workspace holds the slices
    // (after the GroupNorm's own workspace)
    float* kz_ws = nullptr;
    const soar::gn::PwKz kp = soar::gn::pw_kz_plan(N, C_in, C_out, HW, p.chunk, (int)t.pw_kz);
    if (kp.kz > 1) {
        const size_t off = kz_offset(soar::gn::workspace_bytes(p));
        const size_t end = off + soar::gn::pw_kz_bytes(N, C_out, HW, kp.kz);
        if (workspace_bytes >= end) {
            // the slices lie past the GroupNorm part checked above
            if ((rc = check_dev(workspace, end, "workspace"))) return rc;
            kz_ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + off);
        }
    }
    hipError_t e = soar::gn::launch_pw_conv(pa, N, C_in, C_out, HW, p.chunk,
                                            soar::gn::ws_partials(p, workspace), false, 0, kz_ws,
                                            kp.kz, s);
    if (e != hipSuccess) return hip_fail(e, "pointwise convolution launch");
    soar::gn::FwdArgs a{z, gamma, beta, y, mean, rstd, mean_lo, eps, flags, workspace};
    const bool in_apply = residual && !soar::gn::forward_is_small(p, t);
    if (in_apply) {
        a.flags |= SOAR_GN_RESIDUAL;
        a.res = residual;
        if (!aligned16(residual)) p.vec4 = false;
    }
    e = soar::gn::launch_forward_from_partials(p, t, a, s);
    if (e != hipSuccess) return hip_fail(e, "GroupNorm apply launch");
    if (residual && !in_apply) {
        e = soar::gn::launch_add_forward(y, residual, y, oe, s);
        if (e != hipSuccess) return hip_fail(e, "residual add launch");
    }
    return ok();
}

}  // namespace

SOAR_API int soar_pw_conv_gn_silu_forward(const float* x, const float* weight,
                                          const float* bias, const float* gamma,
                                          const float* beta, float* z, float* y, float* mean,
                                          float* rstd, float* mean_lo, int64_t N, int64_t C_in,
                                          int64_t C_out, int64_t HW, int64_t G, float eps,
                                          unsigned flags, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    return pw_conv_gn_forward(x, weight, bias, gamma, beta, nullptr, z, y, mean, rstd, mean_lo,
                              N, C_in, C_out, HW, G, eps, flags, workspace, workspace_bytes,
                              stream);
}

SOAR_API int soar_pw_conv_gn_silu_add_forward(
    const float* x, const float* weight, const float* bias, const float* gamma,
    const float* beta, const float* residual, float* z, float* y, float* mean, float* rstd,
    float* mean_lo, int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t G, float eps,
    unsigned flags, void* workspace, size_t workspace_bytes, void* stream) {
    if (!residual) return fail(SOAR_EINVAL, "residual is NULL");
    return pw_conv_gn_forward(x, weight, bias, gamma, beta, residual, z, y, mean, rstd,
                              mean_lo, N, C_in, C_out, HW, G, eps, flags, workspace,
                              workspace_bytes, stream);
}

SOAR_API size_t soar_pw_conv_backward_workspace_bytes(int64_t N, int64_t C_in, int64_t C_out,
                                                      int64_t HW) {
    int64_t ie = 0, oe = 0;
    if (check_pw_shape(N, C_in, C_out, HW, &ie, &oe) != SOAR_OK || oe == 0 || C_in == 0) {
        g_err.clear();
        return 0;
    }
    const Tuning t = current_tuning();
    const soar::gn::PwBwdPlan p =
        soar::gn::make_pw_bwd_plan(N, C_in, C_out, HW, t.pw_chunk, (int)t.pw_kz, t.pw_wg_waves,
                                   t.pw_wg_target);
    return soar::gn::pw_bwd_workspace_bytes(p);
}

SOAR_API int soar_weight_grad_flush(void* stream) {
    if (soar::gn::weight_finish_pending() == 0) return ok();
    if (static_cast<hipStream_t>(stream) != soar::gn::weight_finish_stream())
        return fail(SOAR_EINVAL,
                    "the pending weight-gradient finishes were queued on another stream");
    const hipError_t e = soar::gn::weight_finish_flush();
    if (e != hipSuccess) return hip_fail(e, "weight-gradient finish launch");
    return ok();
}

SOAR_API size_t soar_weight_grad_pending(void) { return soar::gn::weight_finish_pending(); }

SOAR_API void soar_weight_grad_discard(void) { soar::gn::weight_finish_discard(); }

SOAR_API int soar_pw_conv_backward(const float* dz, const float* x, const float* weight,
                                   float* dx, float* dweight, float* dbias, int64_t N,
                                   int64_t C_in, int64_t C_out, int64_t HW, unsigned flags,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    int64_t ie = 0, oe = 0;
    int rc = check_pw_shape(N, C_in, C_out, HW, &ie, &oe);
    if (rc) return rc;
    if (flags & ~(SOAR_GN_ACCUMULATE_DX | SOAR_DEFER_WEIGHT_FINISH))
        return fail(SOAR_EINVAL,
                    "unsupported flags 0x%x (SOAR_GN_ACCUMULATE_DX, SOAR_DEFER_WEIGHT_FINISH)",
                    flags);
    if (oe == 0 || (!dx && !dweight && !dbias)) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    if ((rc = require_device())) return rc;
    const size_t wb = (size_t)(C_in * C_out) * 4;
    if ((rc = check_dev(dz, (size_t)oe * 4, "dz")) ||
        (dx && (rc = check_dev(weight, wb, "weight"))) ||
        ((dweight) && (rc = check_dev(x, (size_t)ie * 4, "x"))) ||
        (rc = check_dev_opt(dx, (size_t)ie * 4, "dx")) ||
        (rc = check_dev_opt(dweight, wb, "dweight")) ||
        (rc = check_dev_opt(dbias, (size_t)C_out * 4, "dbias")))
        return rc;
    const Tuning t = current_tuning();
    soar::gn::PwBwdPlan p =
        soar::gn::make_pw_bwd_plan(N, C_in, C_out, HW, t.pw_chunk, (int)t.pw_kz, t.pw_wg_waves,
                                   t.pw_wg_target);
    if (!pw_grid_fits(N, HW, p.chunk_dx) || p.Gb > 65535 ||
        p.tiles_co * p.tiles_ci > (int64_t)0x7fffffff)
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    // a workspace sized without the split-K slices (another tuning when it
    // was queried) runs dx without them
    if (p.kz_bytes && workspace_bytes < soar::gn::pw_bwd_workspace_bytes(p))
        p = soar::gn::make_pw_bwd_plan(N, C_in, C_out, HW, t.pw_chunk, 1, t.pw_wg_waves,
                                         t.pw_wg_target);
    const size_t need = soar::gn::pw_bwd_workspace_bytes(p);
    if (workspace_bytes < need)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu this shape needs",
                    workspace_bytes, need);
    if ((rc = check_dev(workspace, need, "workspace"))) return rc;
    soar::gn::PwBwdArgs a{dz, x, weight, dx, dweight, dbias, workspace};
    if ((rc = weight_finish_room(dweight, C_out * C_in, dbias, C_out, stream, flags))) return rc;
    DeferWeightFinish defer((flags & SOAR_DEFER_WEIGHT_FINISH) != 0);
    hipError_t e = soar::gn::launch_pw_backward(p, a, N, C_in, C_out, HW,
                                                (flags & SOAR_GN_ACCUMULATE_DX) != 0,
                                                t.pw_small, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pointwise convolution backward launch");
    return ok();
}

SOAR_API int soar_conv2d_1x1_backward(const float* grad_out, const float* in, const float* weight,
                                      float* grad_in, float* grad_weight, float* grad_bias,
                                      size_t C_in, size_t C_out, size_t HW, void* stream) {
    if (C_in > (size_t)INT64_MAX || C_out > (size_t)INT64_MAX || HW > (size_t)INT64_MAX)
        return fail(SOAR_EINVAL, "dimension too large");
    if (C_out == 0 || HW == 0 || (!grad_in && !grad_weight && !grad_bias)) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    const size_t need =
        soar_pw_conv_backward_workspace_bytes(1, (int64_t)C_in, (int64_t)C_out, (int64_t)HW);
    if (need == 0) {
        int64_t ie = 0, oe = 0;
        int rc = check_pw_shape(1, (int64_t)C_in, (int64_t)C_out, (int64_t)HW, &ie, &oe);
        return rc ? rc : fail(SOAR_EINVAL, "shape is too large");
    }
    int rc = require_device();
    if (rc) return rc;
    void* ws = nullptr;
    if ((rc = owned_workspace(need, &ws, stream))) return rc;
    return soar_pw_conv_backward(grad_out, in, weight, grad_in, grad_weight, grad_bias, 1,
                                 (int64_t)C_in, (int64_t)C_out, (int64_t)HW,
                                 SOAR_GN_ACCUMULATE_DX, ws, need, stream);
}

// ---- depthwise convolution -----------------------------------------------------


}  // extern "C"

namespace {

inline size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of soar_pw_cba_backward.  Fused: the GroupNorm workspace, then
// the weight-gradient block partials.  Unfused: dz, then the GroupNorm
// workspace, then the convolution backward's.
struct CbaLayout {
    bool fused = false;
    Plan gp;
    soar::gn::PwCbaPlan cp;
    size_t gn_bytes = 0, dz_bytes = 0, pw_bytes = 0, fused_bytes = 0, unfused_bytes = 0;
};

bool cba_layout(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t G, const Tuning& t,
                CbaLayout* L) {
    if (!soar::gn::make_plan(N, C_out, HW, G, t, &L->gp)) return false;
    L->gn_bytes = al256(soar::gn::workspace_bytes(L->gp));
    L->dz_bytes = al256((size_t)(N * C_out * HW) * sizeof(float));
    L->pw_bytes = soar_pw_conv_backward_workspace_bytes(N, C_in, C_out, HW);
    L->unfused_bytes = L->dz_bytes + L->gn_bytes + L->pw_bytes;
    L->fused = t.pw_cba_min > 0 && N * HW >= t.pw_cba_min &&
               soar::gn::pw_cba_fused_fits(C_in, C_out, HW);
    if (L->fused) {
        L->cp = soar::gn::make_pw_cba_plan(N, C_in, C_out, HW, t.pw_cba_blocks);
        L->fused = L->cp.blocks <= 0x7fffffff;
        L->fused_bytes = L->gn_bytes + L->cp.part_bytes;
    }
    return true;
}


// Layout of soar_dw_conv_gn_silu_forward's workspace: the GroupNorm
// workspace of the output, then (when the convolution writes the statistics
// partials itself) the tile-group partials.
struct DwGnLayout {
    Plan p;
    soar::gn::DwStatsGeom g;
    bool fused = false;
    size_t gn_bytes = 0, part_bytes = 0;
};

bool dw_gn_layout(const soar::gn::DwShape& sh, int64_t G, const Tuning& t, DwGnLayout* L) {
    if (!soar::gn::make_plan(sh.N, sh.C, sh.Ho * sh.Wo, G, t, &L->p)) return false;
    L->gn_bytes = al256(soar::gn::workspace_bytes(L->p));
    L->fused = !soar::gn::forward_is_small(L->p, t) && soar::gn::dw_stats_geometry(sh, &L->g) &&
               sh.N * sh.C * L->g.tpp <= 0x7fffffff;
    L->part_bytes = L->fused ? al256((size_t)(sh.N * sh.C * L->g.tpp) * sizeof(double2)) : 0;
    return true;
}

}  // namespace

extern "C" {

SOAR_API size_t soar_pw_cba_backward_workspace_bytes(int64_t N, int64_t C_in, int64_t C_out,
                                                     int64_t HW, int64_t G) {
    int64_t ie = 0, oe = 0, elems = 0;
    if (check_pw_shape(N, C_in, C_out, HW, &ie, &oe) != SOAR_OK ||
        check_shape(N, C_out, HW, G, &elems) != SOAR_OK || oe == 0 || C_in == 0) {
        g_err.clear();
        return 0;
    }
    CbaLayout L;
    if (!cba_layout(N, C_in, C_out, HW, G, current_tuning(), &L)) return 0;
    return L.fused ? L.fused_bytes : L.unfused_bytes;
}

SOAR_API int soar_pw_cba_backward(const float* dy, const float* z, const float* x,
                                  const float* weight, const float* gamma, const float* beta,
                                  const float* mean, const float* rstd, const float* mean_lo,
                                  float* dx, float* dweight, float* dgamma, float* dbeta,
                                  int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t G,
                                  unsigned flags, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    int64_t ie = 0, oe = 0, elems = 0;
    int rc = check_pw_shape(N, C_in, C_out, HW, &ie, &oe);
    if (rc) return rc;
    if ((rc = check_shape(N, C_out, HW, G, &elems))) return rc;
    if (flags & ~(SOAR_GN_SILU | SOAR_GN_ACCUMULATE_DX | SOAR_DEFER_WEIGHT_FINISH))
        return fail(SOAR_EINVAL,
                    "unsupported flags 0x%x (SOAR_GN_SILU, SOAR_GN_ACCUMULATE_DX, "
                    "SOAR_DEFER_WEIGHT_FINISH)",
                    flags);
    if ((rc = weight_finish_room(dweight, C_out * C_in, nullptr, 0, stream, flags))) return rc;
    DeferWeightFinish defer((flags & SOAR_DEFER_WEIGHT_FINISH) != 0);
    if (oe == 0 || (!dx && !dweight && !dgamma && !dbeta)) return ok();
    if (C_in == 0) return fail(SOAR_EINVAL, "C_in must be positive");
    if ((rc = require_device())) return rc;
    const Tuning t = current_tuning();
    CbaLayout L;
    if (!cba_layout(N, C_in, C_out, HW, G, t, &L))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!dx && !dweight)  // the parameter gradients alone: the GroupNorm backward
        return soar_gn_silu_backward(dy, z, gamma, beta, mean, rstd, mean_lo, nullptr, dgamma,
                                     dbeta, N, C_out, HW, G, flags & SOAR_GN_SILU, workspace,
                                     workspace_bytes, stream);
    const bool aligned = aligned16(dy) && aligned16(z) && aligned16(x) && aligned16(dx);
    if (L.fused && aligned) {
        const size_t sb = (size_t)(N * G) * sizeof(float), cb = (size_t)C_out * sizeof(float);
        const size_t wb = (size_t)(C_in * C_out) * sizeof(float);
        if ((rc = check_dev(dy, (size_t)oe * 4, "dy")) || (rc = check_dev(z, (size_t)oe * 4, "z")) ||
            (rc = check_dev(x, (size_t)ie * 4, "x")) || (rc = check_dev(weight, wb, "weight")) ||
            (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
            (rc = check_dev_opt(mean_lo, sb, "mean_lo")) ||
            (rc = check_dev_opt(gamma, cb, "gamma")) || (rc = check_dev_opt(beta, cb, "beta")) ||
            (rc = check_dev_opt(dx, (size_t)ie * 4, "dx")) ||
            (rc = check_dev_opt(dweight, wb, "dweight")) ||
            (rc = check_dev_opt(dgamma, cb, "dgamma")) || (rc = check_dev_opt(dbeta, cb, "dbeta")))
            return rc;
        if (workspace_bytes < L.fused_bytes)
            return fail(SOAR_EINVAL,
                        "workspace of %zu bytes is smaller than the %zu this shape needs",
                        workspace_bytes, L.fused_bytes);
        if ((rc = check_dev(workspace, L.fused_bytes, "workspace"))) return rc;
        Plan gp = L.gp;
        gp.vec4 = gp.vec4 && aligned16(z) && aligned16(dy);
        const unsigned gflags = flags & SOAR_GN_SILU;
        soar::gn::BwdArgs a{dy, z, gamma, beta, mean, rstd, mean_lo, nullptr, dgamma, dbeta,
                            gflags, workspace};
        // each block folds the finish of its sample's C_out planes
        soar::gn::BwdSums sums{};
        hipError_t e = soar::gn::launch_backward_sums(
            gp, a, s, &sums, soar::gn::backward_sums_foldable(gp, t, a, C_out));
        if (e != hipSuccess) return hip_fail(e, "GroupNorm backward reduction launch");
        float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + L.gn_bytes);
        soar::gn::PwCbaArgs ca{dy,     z,         x,      weight,          gamma,
                               beta,   mean,      rstd,   sums.mean_lo,    sums.unit_sums,
                               sums.plane_sums, dgamma, dbeta, dx,         dweight,
                               part,   sums.part, sums.cpp};
        e = soar::gn::launch_pw_cba_backward(L.cp, ca, N, C_in, C_out, HW, G, gflags != 0,
                                             (flags & SOAR_GN_ACCUMULATE_DX) != 0, s);
        if (e != hipSuccess) return hip_fail(e, "fused CBA backward launch");
        return ok();
    }
    // the GroupNorm backward into dz (in the workspace), then the
    // convolution backward
    if (workspace_bytes < L.unfused_bytes)
        return fail(SOAR_EINVAL,
                    "workspace of %zu bytes is smaller than the %zu this call needs (%s)",
                    workspace_bytes, L.unfused_bytes,
                    L.fused ? "tensors not 16-byte aligned run the unfused path" : "unfused path");
    char* ws = static_cast<char*>(workspace);
    float* dz = reinterpret_cast<float*>(ws);
    rc = soar_gn_silu_backward(dy, z, gamma, beta, mean, rstd, mean_lo, dz, dgamma, dbeta, N,
                               C_out, HW, G, flags & SOAR_GN_SILU, ws + L.dz_bytes, L.gn_bytes,
                               stream);
    if (rc) return rc;
    return soar_pw_conv_backward(dz, x, weight, dx, dweight, nullptr, N, C_in, C_out, HW,
                                 flags & SOAR_GN_ACCUMULATE_DX, ws + L.dz_bytes + L.gn_bytes,
                                 L.pw_bytes, stream);
}

SOAR_API int soar_dw_conv_forward(const float* x, const float* weight, const float* bias,
                                  float* y, int64_t N, int64_t C, int64_t H_in, int64_t W_in,
                                  int64_t H_out, int64_t W_out, int64_t K, int64_t pad,
                                  int64_t stride, int64_t dil, void* stream) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0;
    int rc = check_dw_shape(sh, &ie, &oe);
    if (rc) return rc;
    if (oe == 0) return ok();
    if ((rc = require_device())) return rc;
    if ((rc = check_dev(y, (size_t)oe * 4, "y")) ||
        (rc = check_dev(weight, (size_t)(C * K * K) * 4, "weight")) ||
        (rc = check_dev_opt(bias, (size_t)C * 4, "bias")) ||
        (ie > 0 && (rc = check_dev(x, (size_t)ie * 4, "x"))))
        return rc;
    if (!dw_grids_fit(sh)) return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    hipError_t e = soar::gn::launch_dw_forward(sh, x, weight, bias, y,
                                               static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "depthwise convolution launch");
}

SOAR_API size_t soar_dw_conv_gn_workspace_bytes(int64_t N, int64_t C, int64_t H_in, int64_t W_in,
                                                int64_t H_out, int64_t W_out, int64_t K,
                                                int64_t pad, int64_t stride, int64_t dil,
                                                int64_t G) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0, elems = 0;
    if (check_dw_shape(sh, &ie, &oe) != SOAR_OK ||
        check_shape(N, C, H_out * W_out, G, &elems) != SOAR_OK || oe == 0) {
        g_err.clear();
        return 0;
    }
    DwGnLayout L;
    if (!dw_gn_layout(sh, G, current_tuning(), &L)) return 0;
    return L.gn_bytes + L.part_bytes;
}

SOAR_API int soar_dw_conv_gn_silu_forward(const float* x, const float* weight, const float* bias,
                                          const float* gamma, const float* beta, float* z,
                                          float* y, float* mean, float* rstd, float* mean_lo,
                                          int64_t N, int64_t C, int64_t H_in, int64_t W_in,
                                          int64_t H_out, int64_t W_out, int64_t K, int64_t pad,
                                          int64_t stride, int64_t dil, int64_t G, float eps,
                                          unsigned flags, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0, elems = 0;
    int rc = check_dw_shape(sh, &ie, &oe);
    if (rc) return rc;
    if ((rc = check_shape(N, C, H_out * W_out, G, &elems))) return rc;
    if (flags & ~SOAR_GN_SILU)
        return fail(SOAR_EINVAL, "unsupported flags 0x%x (SOAR_GN_SILU only)", flags);
    if (!(eps >= 0.0f)) return fail(SOAR_EINVAL, "eps must be >= 0");
    if (oe == 0) return ok();
    if ((rc = require_device())) return rc;
    const size_t sb = (size_t)(N * G) * sizeof(float);
    if ((rc = check_dev(weight, (size_t)(C * K * K) * 4, "weight")) ||
        (rc = check_dev_opt(bias, (size_t)C * 4, "bias")) ||
        (ie > 0 && (rc = check_dev(x, (size_t)ie * 4, "x"))) ||
        (rc = check_dev_opt(gamma, (size_t)C * 4, "gamma")) ||
        (rc = check_dev_opt(beta, (size_t)C * 4, "beta")) ||
        (rc = check_dev(z, (size_t)oe * 4, "z")) || (rc = check_dev(y, (size_t)oe * 4, "y")) ||
        (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
        (rc = check_dev_opt(mean_lo, sb, "mean_lo")))
        return rc;
    if (!dw_grids_fit(sh)) return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    const Tuning t = current_tuning();
    DwGnLayout L;
    if (!dw_gn_layout(sh, G, t, &L))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    L.p.vec4 = L.p.vec4 && aligned16(z) && aligned16(y);
    if ((rc = check_ws(L.p, workspace, workspace_bytes))) return rc;
    if (workspace_bytes < L.gn_bytes + L.part_bytes)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu this call needs",
                    workspace_bytes, L.gn_bytes + L.part_bytes);
    if (L.fused && (rc = check_dev(workspace, L.gn_bytes + L.part_bytes, "workspace")))
        return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    soar::gn::FwdArgs a{z, gamma, beta, y, mean, rstd, mean_lo, eps, flags, workspace};
    if (!L.fused) {
        // no tiled kernel for the shape, or units small enough for the
        // one-launch GroupNorm: the convolution, then the GroupNorm forward
        hipError_t e = soar::gn::launch_dw_forward(sh, x, weight, bias, z, s);
        if (e != hipSuccess) return hip_fail(e, "depthwise convolution launch");
        e = soar::gn::launch_forward(L.p, t, a, s);
        return e == hipSuccess ? ok() : hip_fail(e, "GroupNorm forward launch");
    }
    double2* part = reinterpret_cast<double2*>(static_cast<char*>(workspace) + L.gn_bytes);
    hipError_t e = soar::gn::launch_dw_forward(sh, x, weight, bias, z, s, part);
    if (e != hipSuccess) return hip_fail(e, "depthwise convolution launch");
    e = soar::gn::launch_forward_from_tile_partials(L.p, t, a, part, L.g, H_out, W_out, s);
    return e == hipSuccess ? ok() : hip_fail(e, "GroupNorm finish / apply launch");
}

SOAR_API size_t soar_dw_conv_backward_workspace_bytes(int64_t N, int64_t C, int64_t H_in,
                                                      int64_t W_in, int64_t H_out,
                                                      int64_t W_out, int64_t K, int64_t stride,
                                                      int64_t dil) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, 0, stride, dil);
    int64_t ie = 0, oe = 0;
    if (check_dw_shape(sh, &ie, &oe) != SOAR_OK) {
        g_err.clear();
        return (size_t)-1;
    }
    return soar::gn::dw_bwd_workspace_bytes(sh);
}

SOAR_API int soar_dw_conv_backward(const float* dy, const float* x, const float* weight,
                                   float* dx, float* dweight, float* dbias, int64_t N, int64_t C,
                                   int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out,
                                   int64_t K, int64_t pad, int64_t stride, int64_t dil,
                                   unsigned flags, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0;
    int rc = check_dw_shape(sh, &ie, &oe);
    if (rc) return rc;
    if (flags & ~(SOAR_GN_ACCUMULATE_DX | SOAR_DEFER_WEIGHT_FINISH))
        return fail(SOAR_EINVAL,
                    "unsupported flags 0x%x (SOAR_GN_ACCUMULATE_DX, SOAR_DEFER_WEIGHT_FINISH)",
                    flags);
    if ((!dx && !dweight && !dbias) || N * C == 0) return ok();
    if ((rc = require_device())) return rc;
    const size_t wb = (size_t)(C * K * K) * 4;
    if ((oe > 0 && (rc = check_dev(dy, (size_t)oe * 4, "dy"))) ||
        (dx && ie > 0 && (rc = check_dev(weight, wb, "weight"))) ||
        (dweight && ie > 0 && (rc = check_dev(x, (size_t)ie * 4, "x"))) ||
        (ie > 0 && (rc = check_dev_opt(dx, (size_t)ie * 4, "dx"))) ||
        (rc = check_dev_opt(dweight, wb, "dweight")) ||
        (rc = check_dev_opt(dbias, (size_t)C * 4, "dbias")))
        return rc;
    if (!dw_grids_fit(sh)) return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    const size_t need = (dweight || dbias) ? soar::gn::dw_bwd_workspace_bytes(sh) : 0;
    if (need) {
        if (workspace_bytes < need)
            return fail(SOAR_EINVAL,
                        "workspace of %zu bytes is smaller than the %zu this shape needs",
                        workspace_bytes, need);
        if ((rc = check_dev(workspace, need, "workspace"))) return rc;
    }
    // with no input pixels, dweight gets nothing and dx is empty
    if ((rc = weight_finish_room(dweight, C * K * K, dbias, C, stream, flags))) return rc;
    DeferWeightFinish defer((flags & SOAR_DEFER_WEIGHT_FINISH) != 0);
    hipError_t e = soar::gn::launch_dw_backward(sh, dy, x, weight, ie > 0 ? dx : nullptr,
                                                ie > 0 ? dweight : nullptr, oe > 0 ? dbias : nullptr,
                                                (flags & SOAR_GN_ACCUMULATE_DX) != 0, workspace,
                                                static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "depthwise convolution backward launch");
    return ok();
}

}  // extern "C"

namespace {

// Workspace of soar_dw_cba_backward.  Fused: the GroupNorm workspace, then
// the weight-gradient partials.  Unfused: dz, then the GroupNorm
// workspace, then the depthwise backward's.
struct DwCbaLayout {
    bool fused = false;
    Plan gp;
    size_t gn_bytes = 0, dz_bytes = 0, dw_bytes = 0, fused_bytes = 0, unfused_bytes = 0;
};

bool dw_cba_layout(const soar::gn::DwShape& sh, int64_t G, const Tuning& t, DwCbaLayout* L) {
    const int64_t HWo = sh.Ho * sh.Wo;
    if (!soar::gn::make_plan(sh.N, sh.C, HWo, G, t, &L->gp)) return false;
    L->gn_bytes = al256(soar::gn::workspace_bytes(L->gp));
    L->dz_bytes = al256((size_t)(sh.N * sh.C * HWo) * sizeof(float));
    L->dw_bytes = al256(soar::gn::dw_bwd_workspace_bytes(sh));
    L->unfused_bytes = L->dz_bytes + L->gn_bytes + L->dw_bytes;
    L->fused = t.dw_cba_min > 0 && sh.N * HWo >= t.dw_cba_min && soar::gn::dw_cba_fused_fits(sh) &&
               soar::gn::dw_cba_grid_blocks(sh) <= 0x7fffffff;
    L->fused_bytes = L->fused ? L->gn_bytes + soar::gn::dw_cba_part_bytes(sh) : 0;
    return true;
}

}  // namespace

extern "C" {

SOAR_API size_t soar_dw_cba_backward_workspace_bytes(int64_t N, int64_t C, int64_t H_in,
                                                     int64_t W_in, int64_t H_out, int64_t W_out,
                                                     int64_t K, int64_t pad, int64_t stride,
                                                     int64_t dil, int64_t G) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0, elems = 0;
    if (check_dw_shape(sh, &ie, &oe) != SOAR_OK ||
        check_shape(N, C, H_out * W_out, G, &elems) != SOAR_OK || oe == 0) {
        g_err.clear();
        return 0;
    }
    DwCbaLayout L;
    if (!dw_cba_layout(sh, G, current_tuning(), &L)) return 0;
    return L.fused ? L.fused_bytes : L.unfused_bytes;
}

SOAR_API int soar_dw_cba_backward(const float* dy, const float* z, const float* x,
                                  const float* weight, const float* gamma, const float* beta,
                                  const float* mean, const float* rstd, const float* mean_lo,
                                  float* dx, float* dweight, float* dgamma, float* dbeta,
                                  int64_t N, int64_t C, int64_t H_in, int64_t W_in, int64_t H_out,
                                  int64_t W_out, int64_t K, int64_t pad, int64_t stride,
                                  int64_t dil, int64_t G, unsigned flags, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    const soar::gn::DwShape sh = dw_shape(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil);
    int64_t ie = 0, oe = 0, elems = 0;
    int rc = check_dw_shape(sh, &ie, &oe);
    if (rc) return rc;
    if ((rc = check_shape(N, C, H_out * W_out, G, &elems))) return rc;
    if (flags & ~(SOAR_GN_SILU | SOAR_GN_ACCUMULATE_DX | SOAR_DEFER_WEIGHT_FINISH))
        return fail(SOAR_EINVAL,
                    "unsupported flags 0x%x (SOAR_GN_SILU, SOAR_GN_ACCUMULATE_DX, "
                    "SOAR_DEFER_WEIGHT_FINISH)",
                    flags);
    if ((rc = weight_finish_room(dweight, C * K * K, nullptr, 0, stream, flags))) return rc;
    DeferWeightFinish defer((flags & SOAR_DEFER_WEIGHT_FINISH) != 0);
    if (oe == 0 || (!dx && !dweight && !dgamma && !dbeta)) return ok();
    if ((rc = require_device())) return rc;
    if (!dw_grids_fit(sh)) return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    const Tuning t = current_tuning();
    DwCbaLayout L;
    if (!dw_cba_layout(sh, G, t, &L))
        return fail(SOAR_EINVAL, "shape is too large for one launch grid");
    if (!dx && !dweight)  // the parameter gradients alone: the GroupNorm backward
        return soar_gn_silu_backward(dy, z, gamma, beta, mean, rstd, mean_lo, nullptr, dgamma,
                                     dbeta, N, C, H_out * W_out, G, flags & SOAR_GN_SILU,
                                     workspace, workspace_bytes, stream);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (L.fused) {
        const size_t sb = (size_t)(N * G) * sizeof(float), cb = (size_t)C * sizeof(float);
        const size_t wb = (size_t)(C * K * K) * sizeof(float);
        if ((rc = check_dev(dy, (size_t)oe * 4, "dy")) || (rc = check_dev(z, (size_t)oe * 4, "z")) ||
            (rc = check_dev(x, (size_t)ie * 4, "x")) || (rc = check_dev(weight, wb, "weight")) ||
            (rc = check_dev(mean, sb, "mean")) || (rc = check_dev(rstd, sb, "rstd")) ||
            (rc = check_dev_opt(mean_lo, sb, "mean_lo")) ||
            (rc = check_dev_opt(gamma, cb, "gamma")) || (rc = check_dev_opt(beta, cb, "beta")) ||
            (rc = check_dev_opt(dx, (size_t)ie * 4, "dx")) ||
            (rc = check_dev_opt(dweight, wb, "dweight")) ||
            (rc = check_dev_opt(dgamma, cb, "dgamma")) || (rc = check_dev_opt(dbeta, cb, "dbeta")))
            return rc;
        if (workspace_bytes < L.fused_bytes)
            return fail(SOAR_EINVAL,
                        "workspace of %zu bytes is smaller than the %zu this shape needs",
                        workspace_bytes, L.fused_bytes);
        if ((rc = check_dev(workspace, L.fused_bytes, "workspace"))) return rc;
        Plan gp = L.gp;
        gp.vec4 = gp.vec4 && aligned16(z) && aligned16(dy);
        const unsigned gflags = flags & SOAR_GN_SILU;
        soar::gn::BwdArgs a{dy, z, gamma, beta, mean, rstd, mean_lo, nullptr, dgamma, dbeta,
                            gflags, workspace};
        // each block folds the finish of its unit's C / G planes
        soar::gn::BwdSums sums{};
        hipError_t e = soar::gn::launch_backward_sums(
            gp, a, s, &sums, soar::gn::backward_sums_foldable(gp, t, a, C / G));
        if (e != hipSuccess) return hip_fail(e, "GroupNorm backward reduction launch");
        float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + L.gn_bytes);
        soar::gn::DwCbaArgs da{dy,    z,         x,        weight,       gamma,
                               beta,  mean,      rstd,     sums.mean_lo, sums.unit_sums,
                               sums.plane_sums,  dgamma,   dbeta,        dx,
                               dweight, part,    sums.part, sums.cpp};
        e = soar::gn::launch_dw_cba_backward(sh, da, G, gflags != 0,
                                             (flags & SOAR_GN_ACCUMULATE_DX) != 0, s);
        if (e != hipSuccess) return hip_fail(e, "fused depthwise CBA backward launch");
        return ok();
    }
    // the GroupNorm backward into dz (in the workspace), then the
    // depthwise convolution's backward
    if (workspace_bytes < L.unfused_bytes)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu this call needs",
                    workspace_bytes, L.unfused_bytes);
    char* ws = static_cast<char*>(workspace);
    float* dz = reinterpret_cast<float*>(ws);
    rc = soar_gn_silu_backward(dy, z, gamma, beta, mean, rstd, mean_lo, dz, dgamma, dbeta, N, C,
                               H_out * W_out, G, flags & SOAR_GN_SILU, ws + L.dz_bytes,
                               L.gn_bytes, stream);
    if (rc) return rc;
    return soar_dw_conv_backward(dz, x, weight, dx, dweight, nullptr, N, C, H_in, W_in, H_out,
                                 W_out, K, pad, stride, dil, flags & SOAR_GN_ACCUMULATE_DX,
                                 ws + L.dz_bytes + L.gn_bytes, L.dw_bytes, stream);
}

SOAR_API int soar_conv2d_dw_forward(const float* in, const float* weight, const float* bias,
                                    float* out, size_t C, size_t H_in, size_t W_in,
                                    size_t H_out, size_t W_out, size_t K, size_t pad,
                                    size_t stride, size_t dil, void* stream) {
    const size_t lim = (size_t)1 << 40;
    if (C > lim || H_in > lim || W_in > lim || H_out > lim || W_out > lim || K > lim ||
        pad > lim || stride > lim || dil > lim)
        return fail(SOAR_EINVAL, "dimension too large");
    return soar_dw_conv_forward(in, weight, bias, out, 1, (int64_t)C, (int64_t)H_in,
                                (int64_t)W_in, (int64_t)H_out, (int64_t)W_out, (int64_t)K,
                                (int64_t)pad, (int64_t)stride, (int64_t)dil, stream);
}

SOAR_API int soar_conv2d_dw_backward(const float* grad_out, const float* in, const float* weight,
                                     float* grad_in, float* grad_weight, float* grad_bias,
                                     size_t C, size_t H_in, size_t W_in, size_t H_out,
                                     size_t W_out, size_t K, size_t pad, size_t stride,
                                     size_t dil, void* stream) {
    const size_t lim = (size_t)1 << 40;
    if (C > lim || H_in > lim || W_in > lim || H_out > lim || W_out > lim || K > lim ||
        pad > lim || stride > lim || dil > lim)
        return fail(SOAR_EINVAL, "dimension too large");
    const size_t need = soar_dw_conv_backward_workspace_bytes(
        1, (int64_t)C, (int64_t)H_in, (int64_t)W_in, (int64_t)H_out, (int64_t)W_out, (int64_t)K,
        (int64_t)stride, (int64_t)dil);
    if (need == (size_t)-1) {
        int64_t ie = 0, oe = 0;
        return check_dw_shape(dw_shape(1, (int64_t)C, (int64_t)H_in, (int64_t)W_in,
                                       (int64_t)H_out, (int64_t)W_out, (int64_t)K, (int64_t)pad,
                                       (int64_t)stride, (int64_t)dil),
                              &ie, &oe);
    }
    void* ws = nullptr;
    if (need && (grad_weight || grad_bias)) {
        int rc = require_device();
        if (rc) return rc;
        if ((rc = owned_workspace(need, &ws, stream))) return rc;
    }
    return soar_dw_conv_backward(grad_out, in, weight, grad_in, grad_weight, grad_bias, 1,
                                 (int64_t)C, (int64_t)H_in, (int64_t)W_in, (int64_t)H_out,
                                 (int64_t)W_out, (int64_t)K, (int64_t)pad, (int64_t)stride,
                                 (int64_t)dil, SOAR_GN_ACCUMULATE_DX, ws, need, stream);
}

#define SOAR_ELEMWISE_PRELUDE(n)                                   \
    if ((n) == 0) return ok();                                     \
    if ((size_t)(n) > (size_t)INT64_MAX / 4)                       \
        return fail(SOAR_EINVAL, "element count %zu is too large", (size_t)(n)); \
    {                                                              \
        int rc0 = require_device();                                \
        if (rc0) return rc0;                                       \
    }

SOAR_API int soar_silu_forward(const float* x, float* y, size_t n, void* stream) {
    SOAR_ELEMWISE_PRELUDE(n);
    int rc;
    if ((rc = check_dev(x, n * 4, "x")) || (rc = check_dev(y, n * 4, "y"))) return rc;
    hipError_t e = soar::gn::launch_silu_forward(x, y, (int64_t)n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "silu_forward launch");
}

SOAR_API int soar_silu_backward(const float* grad_y, const float* x, float* grad_x, size_t n,
                                void* stream) {
    SOAR_ELEMWISE_PRELUDE(n);
    int rc;
    if ((rc = check_dev(grad_y, n * 4, "grad_y")) || (rc = check_dev(x, n * 4, "x")) ||
        (rc = check_dev(grad_x, n * 4, "grad_x")))
        return rc;
    hipError_t e = soar::gn::launch_silu_backward(grad_y, x, grad_x, (int64_t)n,
                                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "silu_backward launch");
}

SOAR_API int soar_add_forward(const float* a, const float* b, float* y, size_t n, void* stream) {
    SOAR_ELEMWISE_PRELUDE(n);
    int rc;
    if ((rc = check_dev(a, n * 4, "a")) || (rc = check_dev(b, n * 4, "b")) ||
        (rc = check_dev(y, n * 4, "y")))
        return rc;
    hipError_t e = soar::gn::launch_add_forward(a, b, y, (int64_t)n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "add_forward launch");
}

SOAR_API int soar_add_backward(const float* grad_y, float* grad_a, float* grad_b, size_t n,
                               void* stream) {
    if (!grad_a && !grad_b) return ok();
    SOAR_ELEMWISE_PRELUDE(n);
    int rc;
    if ((rc = check_dev(grad_y, n * 4, "grad_y")) || (rc = check_dev_opt(grad_a, n * 4, "grad_a")) ||
        (rc = check_dev_opt(grad_b, n * 4, "grad_b")))
        return rc;
    hipError_t e = soar::gn::launch_add_backward(grad_y, grad_a, grad_b, (int64_t)n,
                                                 static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "add_backward launch");
}

SOAR_API int soar_fill(float* ptr, float value, size_t n, void* stream) {
    SOAR_ELEMWISE_PRELUDE(n);
    int rc;
    if ((rc = check_dev(ptr, n * 4, "ptr"))) return rc;
    hipError_t e = soar::gn::launch_fill(ptr, value, (int64_t)n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "fill launch");
}

SOAR_API int soar_zero(float* ptr, size_t n, void* stream) { return soar_fill(ptr, 0.0f, n, stream); }

// ---- arena -------------------------------------------------------------------

struct soar_arena {
    void* base = nullptr;
    size_t capacity = 0;
    size_t alignment = 256;
    size_t offset = 0;
    size_t static_boundary = 0;
    size_t live = 0;  // allocations since the last reset (bookkeeping only)
};

SOAR_API int soar_arena_create(size_t capacity_bytes, size_t alignment, soar_arena** arena) {
    if (!arena) return fail(SOAR_EINVAL, "arena out-pointer is NULL");
    *arena = nullptr;
    if (capacity_bytes == 0) return fail(SOAR_EINVAL, "arena capacity must be positive");
    if (alignment == 0 || (alignment & (alignment - 1)))
        return fail(SOAR_EINVAL, "alignment %zu is not a power of two", alignment);
    int rc = require_device();
    if (rc) return rc;
    soar_arena* a = new (std::nothrow) soar_arena;
    if (!a) return fail(SOAR_ENOMEM, "host allocation failed");
    hipError_t e = hipMalloc(&a->base, capacity_bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        delete a;
        return fail(SOAR_ENOMEM, "hipMalloc of %zu arena bytes failed", capacity_bytes);
    }
    a->capacity = capacity_bytes;
    a->alignment = alignment;
    *arena = a;
    return ok();
}

SOAR_API int soar_arena_alloc(soar_arena* a, size_t bytes, void** dptr, size_t* offset) {
    if (!a) return fail(SOAR_EINVAL, "arena is NULL");
    if (bytes == 0) return fail(SOAR_EINVAL, "cannot allocate 0 bytes in the arena");
    const size_t at = (a->offset + a->alignment - 1) & ~(a->alignment - 1);
    if (at < a->offset || at > a->capacity || a->capacity - at < bytes)
        return fail(SOAR_ENOMEM, "arena capacity exceeded (%zu + %zu > %zu)", at, bytes,
                    a->capacity);
    a->offset = at + bytes;
    a->live += 1;
    if (dptr) *dptr = static_cast<char*>(a->base) + at;
    if (offset) *offset = at;
    return ok();
}

SOAR_API int soar_arena_freeze_static(soar_arena* a) {
    if (!a) return fail(SOAR_EINVAL, "arena is NULL");
    const size_t b = (a->offset + a->alignment - 1) & ~(a->alignment - 1);
    a->static_boundary = b < a->capacity ? b : a->capacity;
    a->offset = a->static_boundary;
    a->live = 0;
    return ok();
}

SOAR_API int soar_arena_reset_dynamic(soar_arena* a) {
    if (!a) return fail(SOAR_EINVAL, "arena is NULL");
    a->offset = a->static_boundary;
    a->live = 0;
    return ok();
}

SOAR_API int soar_arena_info(const soar_arena* a, size_t* capacity, size_t* current_offset,
                             size_t* static_boundary, void** base) {
    if (!a) return fail(SOAR_EINVAL, "arena is NULL");
    if (capacity) *capacity = a->capacity;
    if (current_offset) *current_offset = a->offset;
    if (static_boundary) *static_boundary = a->static_boundary;
    if (base) *base = a->base;
    return ok();
}

SOAR_API int soar_arena_destroy(soar_arena* a) {
    if (!a) return ok();
    hipError_t e = hipFree(a->base);
    delete a;
    if (e != hipSuccess) return hip_fail(e, "hipFree(arena)");
    return ok();
}

SOAR_API int soar_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!src) return fail(SOAR_EINVAL, "src is NULL");
    int rc = require_device();
    if (rc || (rc = check_dev(dst, bytes, "dst"))) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? ok() : hip_fail(e, "host-to-device copy");
}

SOAR_API int soar_memcpy_async(void* dst, const void* src, size_t bytes, int kind,
                               void* stream) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(SOAR_EINVAL, "dst and src must not be NULL");
    if (kind < 0 || kind > 2) return fail(SOAR_EINVAL, "kind must be 0, 1 or 2");
    int rc = require_device();
    if (rc) return rc;
    if (kind != 1 && (rc = check_dev(dst, bytes, "dst"))) return rc;  // (kind 1: dst is host)
    if (kind != 0 && (rc = check_dev(src, bytes, "src"))) return rc;  // (kind 0: src is host)
    static const hipMemcpyKind kinds[3] = {hipMemcpyHostToDevice, hipMemcpyDeviceToHost,
                                           hipMemcpyDeviceToDevice};
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kinds[kind], static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "asynchronous copy");
}

SOAR_API int soar_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!dst) return fail(SOAR_EINVAL, "dst is NULL");
    int rc = require_device();
    if (rc || (rc = check_dev(src, bytes, "src"))) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? ok() : hip_fail(e, "device-to-host copy");
}

SOAR_API int soar_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return ok();
    int rc = require_device();
    if (rc || (rc = check_dev(dst, bytes, "dst")) || (rc = check_dev(src, bytes, "src"))) return rc;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "device-to-device copy");
}

// ---- timing ------------------------------------------------------------------

SOAR_API int soar_prof_enable(int on) {
    g_prof_on.store(on != 0);
    return ok();
}

SOAR_API int soar_prof_summary(char* buf, size_t buflen) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    struct Agg {
        std::string name;
        long launches;
        double ms;
    };
    std::vector<Agg> agg;
    hipError_t first_err = hipSuccess;
    for (ProfRec& r : g_prof) {
        float ms = 0.0f;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
        if (e != hipSuccess && first_err == hipSuccess) first_err = e;
        auto it = std::find_if(agg.begin(), agg.end(),
                               [&](const Agg& a) { return a.name == r.name; });
        if (it == agg.end()) agg.push_back({r.name, 1, (double)ms});
        else {
            it->launches += 1;
            it->ms += ms;
        }
        g_event_pool.push_back(r.start);
        g_event_pool.push_back(r.stop);
    }
    g_prof.clear();
    if (first_err != hipSuccess) {
        (void)hipGetLastError();
        return hip_fail(first_err, "reading kernel timing events");
    }
    std::string js = "[";
    for (size_t i = 0; i < agg.size(); ++i) {
        char item[256];
        std::snprintf(item, sizeof item, "%s{\"kernel\":\"%s\",\"launches\":%ld,\"total_ms\":%.6f}",
                      i ? "," : "", agg[i].name.c_str(), agg[i].launches, agg[i].ms);
        js += item;
    }
    js += "]";
    if (buf && buflen) {
        std::strncpy(buf, js.c_str(), buflen - 1);
        buf[buflen - 1] = '\0';
    }
    g_err.clear();
    return (int)agg.size();
}

SOAR_API int soar_gn_tune(int key, int64_t value) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    switch (key) {
        case SOAR_TUNE_CHUNK:
            if (value < 1024 || value % 1024 || value > (1 << 24))
                return fail(SOAR_EINVAL, "chunk must be a multiple of 1024 in [1024, 2^24]");
            g_tune.chunk = value;
            return ok();
        case SOAR_TUNE_CHUNK2:
            if (value < 1024 || value % 1024 || value > (1 << 24))
                return fail(SOAR_EINVAL, "chunk2 must be a multiple of 1024 in [1024, 2^24]");
            g_tune.chunk2 = value;
            return ok();
        case SOAR_TUNE_REVERSE:
            if (value != 0 && value != 1) return fail(SOAR_EINVAL, "reverse must be 0 or 1");
            g_tune.reverse = (int)value;
            return ok();
        case SOAR_TUNE_NT_STORE:
            if (value != 0 && value != 1) return fail(SOAR_EINVAL, "nt_store must be 0 or 1");
            g_tune.nt_store = (int)value;
            return ok();
        case SOAR_TUNE_BATCH_MB:
            if (value < 0 || value > (1 << 20))
                return fail(SOAR_EINVAL, "batch_mb must be in [0, 2^20]");
            g_tune.batch_mb = value;
            return ok();
        case SOAR_TUNE_STREAMS:
            if (value != 1 && value != 2) return fail(SOAR_EINVAL, "streams must be 1 or 2");
            g_tune.streams = (int)value;
            return ok();
        case SOAR_TUNE_NT_LOAD:
            if (value < 0 || value > 3)
                return fail(SOAR_EINVAL, "nt_load must be 0..3 (bit 0: second passes, bit 1: first passes)");
            g_tune.nt_load = (int)value;
            return ok();
        case SOAR_TUNE_PW_CHUNK:
            if (value < 128 || value % 128 || value > (1 << 20))
                return fail(SOAR_EINVAL, "pw_chunk must be a multiple of 128 in [128, 2^20]");
            g_tune.pw_chunk = value;
            return ok();
        case SOAR_TUNE_SMALL_UNIT:
            if (value < 0 || value > (1 << 20))
                return fail(SOAR_EINVAL, "small_unit must be in [0, 2^20]");
            g_tune.small_unit = value;
            return ok();
        case SOAR_TUNE_FOLD_MAX:
            if (value < 0 || value > 4096)
                return fail(SOAR_EINVAL, "fold_max must be in [0, 4096]");
            g_tune.fold_max = value;
            return ok();
        case SOAR_TUNE_PW_SMALL:
            if (value < 0 || value > ((int64_t)1 << 40))
                return fail(SOAR_EINVAL, "pw_small must be in [0, 2^40]");
            g_tune.pw_small = value;
            return ok();
        case SOAR_TUNE_PW_SPLITK:
            if (value < 1 || value > 8) return fail(SOAR_EINVAL, "pw_splitk must be in [1, 8]");
            g_tune.pw_kz = value;
            return ok();
        case SOAR_TUNE_LOADS:
            if (value != 4 && value != 8) return fail(SOAR_EINVAL, "loads must be 4 or 8");
            g_tune.loads = (int)value;
            return ok();
        case SOAR_TUNE_PW_WG_WAVES:
            if (value != 1 && value != 2 && value != 4 && value != 8)
                return fail(SOAR_EINVAL, "pw_wg_waves must be 1, 2, 4 or 8");
            g_tune.pw_wg_waves = (int)value;
            return ok();
        case SOAR_TUNE_PW_WG_TARGET:
            if (value < 256 || value > (1 << 20))
                return fail(SOAR_EINVAL, "pw_wg_target must be in [256, 2^20]");
            g_tune.pw_wg_target = value;
            return ok();
        case SOAR_TUNE_PW_CBA_MIN:
            if (value < 0 || value > ((int64_t)1 << 40))
                return fail(SOAR_EINVAL, "pw_cba_min must be in [0, 2^40]");
            g_tune.pw_cba_min = value;
            return ok();
        case SOAR_TUNE_PW_CBA_BLOCKS:
            if (value < 64 || value > (1 << 20))
                return fail(SOAR_EINVAL, "pw_cba_blocks must be in [64, 2^20]");
            g_tune.pw_cba_blocks = value;
            return ok();
        case SOAR_TUNE_DW_CBA_MIN:
            if (value < 0 || value > ((int64_t)1 << 40))
                return fail(SOAR_EINVAL, "dw_cba_min must be in [0, 2^40]");
            g_tune.dw_cba_min = value;
            return ok();
        case SOAR_TUNE_NT_TAIL_MB:
            if (value < 0 || value > (1 << 20))
                return fail(SOAR_EINVAL, "nt_tail_mb must be in [0, 2^20]");
            g_tune.nt_tail_mb = value;
            return ok();
        default:
            return fail(SOAR_EINVAL, "unknown tuning key %d", key);
    }
}

SOAR_API int64_t soar_gn_tune_get(int key) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    switch (key) {
        case SOAR_TUNE_CHUNK: return g_tune.chunk;
        case SOAR_TUNE_CHUNK2: return g_tune.chunk2;
        case SOAR_TUNE_REVERSE: return g_tune.reverse;
        case SOAR_TUNE_NT_STORE: return g_tune.nt_store;
        case SOAR_TUNE_BATCH_MB: return g_tune.batch_mb;
        case SOAR_TUNE_STREAMS: return g_tune.streams;
        case SOAR_TUNE_NT_LOAD: return g_tune.nt_load;
        case SOAR_TUNE_PW_CHUNK: return g_tune.pw_chunk;
        case SOAR_TUNE_SMALL_UNIT: return g_tune.small_unit;
        case SOAR_TUNE_PW_SMALL: return g_tune.pw_small;
        case SOAR_TUNE_FOLD_MAX: return g_tune.fold_max;
        case SOAR_TUNE_PW_SPLITK: return g_tune.pw_kz;
        case SOAR_TUNE_LOADS: return g_tune.loads;
        case SOAR_TUNE_PW_WG_WAVES: return g_tune.pw_wg_waves;
        case SOAR_TUNE_PW_WG_TARGET: return g_tune.pw_wg_target;
        case SOAR_TUNE_PW_CBA_MIN: return g_tune.pw_cba_min;
        case SOAR_TUNE_PW_CBA_BLOCKS: return g_tune.pw_cba_blocks;
        case SOAR_TUNE_DW_CBA_MIN: return g_tune.dw_cba_min;
        case SOAR_TUNE_NT_TAIL_MB: return g_tune.nt_tail_mb;
        default: return -1;
    }
}

}  // extern "C"
