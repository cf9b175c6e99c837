// noalloc.hip - soar_group_norm_backward_noalloc: the reference-signature
// GroupNorm backward without any allocation, for callers that cannot call
// hipMalloc (code under HIP graph capture, tight serving loops, harnesses
// that forbid it).
//
// soar_group_norm_backward keeps a library-owned workspace that it grows
// with hipFree / hipMalloc.  This variant runs the same kernels with their
// workspace (chunk partials, plane and unit sums, mean residuals) in the
// file-scope device array `scratch` below, of kScratchBytes per device,
// held until the process ends.
//
// Host code never passes `scratch` itself to a kernel or a copy: in host
// code that name stands for a host-side shadow, not a device address.  The
// device address comes from hipGetSymbolAddress, called once per device with
// that device current, at the library's set-up there (require_device(), the
// start of every entry point's first call on the device; so a caller that
// has made any call on a device before it captures a graph runs no lookup
// inside the capture), and is kept per device.  The lookup switches the
// thread to relaxed capture mode, so even a first call made under capture
// may load the scratch's code object.
//
// Every call on one device shares that device's array and leaves its
// contents behind; no region needs to start at zero (each call writes every
// workspace word it reads before reading it).  Calls that overlap in time on
// one device (other streams, other threads) race on the array.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "capi_common.hpp"
#include "soar_gn.h"

namespace {

constexpr size_t kScratchBytes = SOAR_GN_NOALLOC_SCRATCH_BYTES;  // per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace soar::capi {

hipError_t noalloc_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
            (void)hipThreadExchangeStreamCaptureMode(&mode);
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            (void)hipThreadExchangeStreamCaptureMode(&mode);  // the caller's mode back
            if (e != hipSuccess || !p) {
                (void)hipGetLastError();
                return e != hipSuccess ? e : hipErrorInvalidSymbol;
            }
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace soar::capi

extern "C" {

SOAR_API int soar_group_norm_backward_noalloc(const float* grad_out, const float* in,
                                              const float* gamma, const float* saved_mean,
                                              const float* saved_rstd, float* grad_in,
                                              float* grad_gamma, float* grad_beta,
                                              size_t num_groups, size_t C, size_t HW,
                                              void* stream) {
    using namespace soar::capi;
    if (C == 0 || HW == 0) return ok();
    if (num_groups == 0 || C % num_groups)
        return fail(SOAR_EINVAL, "C=%zu is not divisible by num_groups=%zu", C, num_groups);
    if (C > (size_t)INT64_MAX || HW > (size_t)INT64_MAX)
        return fail(SOAR_EINVAL, "shape is too large");
    int rc = require_device();
    if (rc) return rc;
    const size_t need =
        soar_gn_workspace_bytes(1, (int64_t)C, (int64_t)HW, (int64_t)num_groups);
    if (need == 0) return fail(SOAR_EINVAL, "shape is too large");
    if (need > kScratchBytes)
        return fail(SOAR_EINVAL,
                    "C=%zu HW=%zu needs %zu bytes of workspace; the static scratch holds %zu "
                    "(use soar_group_norm_backward)",
                    C, HW, need, kScratchBytes);
    void* ws = nullptr;
    const hipError_t e = noalloc_scratch(&ws);
    if (e != hipSuccess)
        return fail(SOAR_EHIP, "hipGetSymbolAddress(scratch): %s (%d)", hipGetErrorString(e),
                    (int)e);
    return gn_backward(grad_out, in, gamma, nullptr, saved_mean, saved_rstd, nullptr, grad_in,
                       grad_gamma, grad_beta, 1, (int64_t)C, (int64_t)HW, (int64_t)num_groups,
                       SOAR_GN_ACCUMULATE_DX, ws, kScratchBytes, stream, true);
}

}  // extern "C"
