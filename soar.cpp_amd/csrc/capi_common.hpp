// capi_common.hpp - validation and status helpers shared by the C-ABI
// translation units of libsoar_gn.so (capi.cpp, ops_capi.cpp).
//
// Every entry point returns SOAR_OK or a negative SOAR_E* status and leaves
// a message for soar_last_error() on the calling thread.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace soar::capi {

extern thread_local std::string g_err;

// Records a printf-style message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns SOAR_OK.
int ok();
int hip_fail(hipError_t e, const char* what);
int device_count();
// SOAR_ENODEV when no HIP device is visible.  Also the library's set-up on
// the current device: its first call there resolves the device address of
// soar_group_norm_backward_noalloc's static scratch (noalloc_scratch), so a
// caller that has made any call on a device before capturing a graph runs
// no symbol lookup inside the capture.
int require_device();
// Resolves (once per device) the current device's address of the static
// scratch behind soar_group_norm_backward_noalloc; hipSuccess or the error
// of the lookup.  Records no error message.
hipError_t noalloc_scratch(void** out);
// `p` must be device memory with at least `bytes` bytes from p to the end
// of its allocation (a host pointer or a too-short buffer is rejected here
// rather than faulting the GPU).
int check_dev(const void* p, size_t bytes, const char* name);
// Same, a null pointer allowed.
int check_dev_opt(const void* p, size_t bytes, const char* name);
bool aligned16(const void* p);
// Library-owned workspace of the current device, grown to `need` bytes
// (used by the entry points with the reference's workspace-free
// signatures).  Callers on one device share it.  Growing it would call
// hipFree / hipMalloc, so while `stream` is being captured into a graph a
// grow is refused with SOAR_EINVAL instead (a capture may reuse a buffer
// that an earlier call outside the capture already grew).
int owned_workspace(size_t need, void** out, void* stream);

// Validation and launch of the fused GroupNorm(+SiLU) backward
// (soar_gn_silu_backward).  ws_scratch: `workspace` is the library's static
// device scratch of `workspace_bytes` bytes, so it is not looked up as an
// allocation, and the call creates nothing (one stream, no timing events).
int gn_backward(const float* dy, const float* x, const float* gamma, const float* beta,
                const float* mean, const float* rstd, const float* mean_lo, float* dx,
                float* dgamma, float* dbeta, int64_t N, int64_t C, int64_t HW, int64_t G,
                unsigned flags, void* workspace, size_t workspace_bytes, void* stream,
                bool ws_scratch);
// Set while a ws_scratch call runs on this thread: kernel timing is skipped.
extern thread_local bool g_quiet_call;

// For the duration of one convolution backward call: with `on` its weight-
// gradient finishes are queued on the thread (SOAR_DEFER_WEIGHT_FINISH)
// instead of launched.  Nested calls (a CBA backward's convolution
// backward) keep an enclosing call's setting.
class DeferWeightFinish {
public:
    explicit DeferWeightFinish(bool on);
    ~DeferWeightFinish();
    DeferWeightFinish(const DeferWeightFinish&) = delete;
    DeferWeightFinish& operator=(const DeferWeightFinish&) = delete;

private:
    bool prev_;
};
// Before a convolution backward call launches: runs the queued finishes
// when they add into this call's dweight / dbias, or when a deferring call
// comes on another stream (SOAR_OK, or the launch's error status).
int weight_finish_room(const float* dweight, int64_t nw, const float* dbias, int64_t nb,
                       void* stream, unsigned flags);

}  // namespace soar::capi
