// ops_capi.cpp - the C-ABI of the model operators (declared in
// include/soar_ops.h): argument validation, then the launchers of
// model_ops.hip.  Same conventions as capi.cpp: empty input is SOAR_OK with
// no launch; every failure is a negative status with a message; device
// buffers are checked against their allocations before anything launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "capi_common.hpp"
#include "gn_internal.hpp"
#include "ops_internal.hpp"
#include "soar_ops.h"

using namespace soar::capi;
using soar::ops::ConvShape;

namespace {

hipStream_t S(void* stream) { return static_cast<hipStream_t>(stream); }

int launched(hipError_t e, const char* what) { return e == hipSuccess ? ok() : hip_fail(e, what); }

// a*b*... without overflow, below 2^62 / 4 bytes.
bool mul_ok(std::initializer_list<int64_t> f, int64_t* out) {
    int64_t p = 1;
    for (int64_t v : f) {
        if (v < 0 || __builtin_mul_overflow(p, v, &p)) return false;
    }
    if (p > INT64_MAX / 8) return false;
    *out = p;
    return true;
}

int check_count(size_t n) {
    if (n > (size_t)INT64_MAX / 8) return fail(SOAR_EINVAL, "element count %zu is too large", n);
    return require_device();
}

// ---- convolution ----------------------------------------------------------
int check_conv(const ConvShape& c, int64_t* in_e, int64_t* out_e, int64_t* w_e) {
    if (c.N < 0 || c.C_in <= 0 || c.C_out <= 0 || c.H <= 0 || c.W <= 0 || c.Ho <= 0 ||
        c.Wo <= 0 || c.K <= 0 || c.pad < 0 || c.S <= 0 || c.D <= 0 || c.groups <= 0)
        return fail(SOAR_EINVAL, "convolution: invalid size, kernel, stride, dilation or groups");
    if (c.C_in % c.groups || c.C_out % c.groups)
        return fail(SOAR_EINVAL, "convolution: C_in=%lld and C_out=%lld must be multiples of groups=%lld",
                    (long long)c.C_in, (long long)c.C_out, (long long)c.groups);
    // output size of layers.cpp:330-332
    const int64_t ek = c.D * (c.K - 1) + 1;
    if (c.H + 2 * c.pad < ek || c.W + 2 * c.pad < ek ||
        c.Ho != (c.H + 2 * c.pad - ek) / c.S + 1 || c.Wo != (c.W + 2 * c.pad - ek) / c.S + 1)
        return fail(SOAR_EINVAL,
                    "convolution: output %lldx%lld does not match input %lldx%lld with K=%lld "
                    "pad=%lld stride=%lld dil=%lld",
                    (long long)c.Ho, (long long)c.Wo, (long long)c.H, (long long)c.W,
                    (long long)c.K, (long long)c.pad, (long long)c.S, (long long)c.D);
    if (!mul_ok({c.N, c.C_in, c.H, c.W}, in_e) || !mul_ok({c.N, c.C_out, c.Ho, c.Wo}, out_e) ||
        !mul_ok({c.C_out, c.C_in / c.groups, c.K, c.K}, w_e))
        return fail(SOAR_EINVAL, "convolution: tensor sizes overflow");
    int64_t rows = 0;
    if (!mul_ok({c.C_out, c.C_in / c.groups, c.K * c.K + 1}, &rows) || rows > INT32_MAX ||
        (c.N * c.Ho * c.Wo) / 16384 >= 65535)
        return fail(SOAR_EINVAL, "convolution: too many weight taps or output positions for the "
                                 "weight-gradient grid");
    return SOAR_OK;
}

int conv_forward(const float* x, const float* w, const float* b, float* y, const ConvShape& c,
                 void* stream) {
    int64_t ie, oe, we;
    int rc;
    if ((rc = check_conv(c, &ie, &oe, &we))) return rc;
    if (c.N == 0) return ok();
    if ((rc = require_device())) return rc;
    if ((rc = check_dev(x, ie * 4, "in")) || (rc = check_dev(w, we * 4, "weight")) ||
        (rc = check_dev_opt(b, c.C_out * 4, "bias")) || (rc = check_dev(y, oe * 4, "out")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "conv_general_fwd");
    hipError_t e = soar::ops::launch_conv_forward(x, w, b, y, c, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "conv2d_forward launch");
}

int conv_backward(const float* dy, const float* x, const float* w, float* dx, float* dw,
                  float* db, const ConvShape& c, bool acc_dx, void* ws, size_t ws_bytes,
                  void* stream) {
    int64_t ie, oe, we;
    int rc;
    if ((rc = check_conv(c, &ie, &oe, &we))) return rc;
    if (c.N == 0 || (!dx && !dw && !db)) return ok();
    if ((rc = require_device())) return rc;
    if ((rc = check_dev(dy, oe * 4, "grad_out")) || (rc = check_dev(w, we * 4, "weight")) ||
        (rc = check_dev_opt(dx, ie * 4, "grad_in")) ||
        (rc = check_dev_opt(dw, we * 4, "grad_weight")) ||
        (rc = check_dev_opt(db, c.C_out * 4, "grad_bias")))
        return rc;
    if (dw || db) {
        if ((rc = check_dev(x, ie * 4, "in"))) return rc;
        const size_t need = soar::ops::conv_backward_workspace_bytes(c);
        if (ws_bytes < need)
            return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu needed",
                        ws_bytes, need);
        if ((rc = check_dev(ws, need, "workspace"))) return rc;
    }
    const int tok = soar::gn::prof_begin(S(stream), "conv_general_bwd");
    hipError_t e =
        soar::ops::launch_conv_backward(dy, x, w, dx, dw, db, c, acc_dx, ws, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "conv2d_backward launch");
}

ConvShape conv_shape(int64_t N, int64_t C_in, int64_t C_out, int64_t H, int64_t W, int64_t Ho,
                     int64_t Wo, int64_t K, int64_t pad, int64_t stride, int64_t dil,
                     int64_t groups) {
    return ConvShape{N, C_in, C_out, H, W, Ho, Wo, K, pad, stride, dil, groups};
}

bool fits_i64(std::initializer_list<size_t> v) {
    for (size_t x : v)
        if (x > (size_t)INT64_MAX / 8) return false;
    return true;
}

// ---- per-plane operators ----------------------------------------------------
int check_planes(size_t C, size_t HW, int64_t* n) {
    if (!fits_i64({C, HW}) || !mul_ok({(int64_t)C, (int64_t)HW}, n))
        return fail(SOAR_EINVAL, "C*HW overflows");
    return SOAR_OK;
}

int resize_check(const float* src, const float* dst, size_t C, size_t H_in, size_t W_in,
                 size_t H_out, size_t W_out, bool backward) {
    int64_t ni, no;
    if (!fits_i64({C, H_in, W_in, H_out, W_out}) ||
        !mul_ok({(int64_t)C, (int64_t)H_in, (int64_t)W_in}, &ni) ||
        !mul_ok({(int64_t)C, (int64_t)H_out, (int64_t)W_out}, &no))
        return fail(SOAR_EINVAL, "upsample: sizes overflow");
    if (H_in == 0 || W_in == 0 || H_out == 0 || W_out == 0)
        return fail(SOAR_EINVAL, "upsample: empty input or output plane");
    if (std::max({H_in, W_in, H_out, W_out}) > (size_t)INT32_MAX)
        return fail(SOAR_EINVAL, "upsample: a plane side exceeds 2^31 - 1");
    int rc;
    if ((rc = require_device())) return rc;
    if (backward)
        return (rc = check_dev(src, no * 4, "grad_out")) ? rc : check_dev(dst, ni * 4, "grad_in");
    return (rc = check_dev(src, ni * 4, "in")) ? rc : check_dev(dst, no * 4, "out");
}

// ---- losses -------------------------------------------------------------------
// Sums of the Dice+BCE loss (fp64: bce, inter, sum_p, sum_y), synchronous.
int loss_sums(const float* z, const float* y, size_t n, float pos_weight, double out[4],
              void* stream) {
    int rc;
    if ((rc = check_count(n))) return rc;
    if ((rc = check_dev(z, n * 4, "logits")) || (rc = check_dev(y, n * 4, "targets"))) return rc;
    const size_t need = soar::ops::loss_sums_workspace_bytes((int64_t)n);
    void* ws = nullptr;
    if ((rc = owned_workspace(need, &ws, stream))) return rc;
    // the partials first, the 4 results at the end of the same buffer
    double* res = static_cast<double*>(ws) + (need / sizeof(double) - 4);
    const int tok = soar::gn::prof_begin(S(stream), "dice_bce_sums");
    hipError_t e = soar::ops::launch_loss_sums(z, y, (int64_t)n, pos_weight, res, ws, S(stream));
    soar::gn::prof_end(S(stream), tok);
    if (e != hipSuccess) return hip_fail(e, "loss sums launch");
    e = hipMemcpyAsync(out, res, 4 * sizeof(double), hipMemcpyDeviceToHost, S(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(S(stream));
    return e == hipSuccess ? ok() : hip_fail(e, "loss sums read-back");
}

// BCE (weight 1) and Dice (weight 1) values from the sums, as
// loss_kernels.cu:51-69 and :141-174 finish them (the dice statistics are
// handed on as fp32, as the reference returns them).
void finish_losses(const double s[4], size_t n, float pos_weight_unused, float smooth,
                   float* bce, float* dice, float* inter, float* sum_p, float* sum_y) {
    (void)pos_weight_unused;
    *bce = (float)(1.0 * (s[0] / (double)n));
    *inter = (float)s[1];
    *sum_p = (float)s[2];
    *sum_y = (float)s[3];
    const double denom = (double)*sum_p + (double)*sum_y + (double)smooth;
    const double numer = 2.0 * (double)*inter + (double)smooth;
    *dice = (float)(1.0 * (1.0 - numer / (denom + 1e-7)));
}

// Flags of the _ex backward entry points: SOAR_GN_ACCUMULATE_DX adds into
// the gradient outputs, 0 writes them.  *acc receives the choice.
int grad_flags(unsigned flags, const char* what, bool* acc) {
    if (flags & ~SOAR_GN_ACCUMULATE_DX)
        return fail(SOAR_EINVAL, "%s: unsupported flags 0x%x (SOAR_GN_ACCUMULATE_DX only)", what,
                    flags);
    *acc = (flags & SOAR_GN_ACCUMULATE_DX) != 0;
    return SOAR_OK;
}

int loss_bwd(const float* z, const float* y, float* gz, size_t n, float go, float w, float bw,
             float dw, float pw, float smooth, float inter, float sum_p, float sum_y,
             void* stream, bool acc = true) {
    if (n == 0) return ok();
    int rc;
    if ((rc = check_count(n))) return rc;
    if ((rc = check_dev(z, n * 4, "logits")) || (rc = check_dev(y, n * 4, "targets")) ||
        (rc = check_dev(gz, n * 4, "grad_logits")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "dice_bce_bwd");
    hipError_t e = soar::ops::launch_dice_bce_backward(z, y, gz, (int64_t)n, go, w, bw, dw, pw,
                                                       smooth, inter, sum_p, sum_y, acc,
                                                       S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "loss backward launch");
}

// ---- multi-tensor table of the host-array entry point -------------------------
struct TableBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_table_mu;
std::vector<TableBuf> g_tables;

int table_buffer(size_t need, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_table_mu);
    if ((int)g_tables.size() <= dev) g_tables.resize(dev + 1);
    TableBuf& t = g_tables[dev];
    if (t.bytes < need) {
        if (t.ptr) {
            e = hipFree(t.ptr);
            t.ptr = nullptr;
            t.bytes = 0;
            if (e != hipSuccess) return hip_fail(e, "hipFree(tensor table)");
        }
        e = hipMalloc(&t.ptr, need);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            t.ptr = nullptr;
            return fail(SOAR_ENOMEM, "hipMalloc of a %zu-byte tensor table failed", need);
        }
        t.bytes = need;
    }
    *out = t.ptr;
    return SOAR_OK;
}

int check_table(const void* arr, int n_tensors, const char* name) {
    if (n_tensors > soar::ops::kMaxMultiTensors)
        return fail(SOAR_EINVAL, "%d tensors exceed the multi-tensor limit of %d", n_tensors,
                    soar::ops::kMaxMultiTensors);
    return check_dev(arr, (size_t)n_tensors * 8, name);
}

}  // namespace

extern "C" {

// ---- convolution --------------------------------------------------------------
SOAR_API int soar_conv2d_forward(const float* in, const float* weight, const float* bias,
                                 float* out, size_t C_in, size_t C_out, size_t H_in,
                                 size_t W_in, size_t H_out, size_t W_out, size_t K, size_t pad,
                                 size_t stride, size_t dil, size_t groups, void* stream) {
    if (!fits_i64({C_in, C_out, H_in, W_in, H_out, W_out, K, pad, stride, dil, groups}))
        return fail(SOAR_EINVAL, "conv2d_forward: argument too large");
    return conv_forward(in, weight, bias, out,
                        conv_shape(1, C_in, C_out, H_in, W_in, H_out, W_out, K, pad, stride,
                                   dil, groups),
                        stream);
}

SOAR_API int soar_conv2d_backward(const float* grad_out, const float* in, const float* weight,
                                  float* grad_in, float* grad_weight, float* grad_bias,
                                  size_t C_in, size_t C_out, size_t H_in, size_t W_in,
                                  size_t H_out, size_t W_out, size_t K, size_t pad,
                                  size_t stride, size_t dil, size_t groups, void* stream) {
    if (!fits_i64({C_in, C_out, H_in, W_in, H_out, W_out, K, pad, stride, dil, groups}))
        return fail(SOAR_EINVAL, "conv2d_backward: argument too large");
    const ConvShape c =
        conv_shape(1, C_in, C_out, H_in, W_in, H_out, W_out, K, pad, stride, dil, groups);
    int64_t ie, oe, we;
    int rc;
    if ((rc = check_conv(c, &ie, &oe, &we))) return rc;
    void* ws = nullptr;
    size_t need = 0;
    if (grad_weight || grad_bias) {
        if ((rc = require_device())) return rc;
        need = soar::ops::conv_backward_workspace_bytes(c);
        if ((rc = owned_workspace(need, &ws, stream))) return rc;
    }
    return conv_backward(grad_out, in, weight, grad_in, grad_weight, grad_bias, c, true, ws,
                         need, stream);
}

SOAR_API int soar_conv_forward(const float* x, const float* weight, const float* bias, float* y,
                               int64_t N, int64_t C_in, int64_t C_out, int64_t H, int64_t W,
                               int64_t Ho, int64_t Wo, int64_t K, int64_t pad, int64_t stride,
                               int64_t dil, int64_t groups, void* stream) {
    return conv_forward(x, weight, bias, y,
                        conv_shape(N, C_in, C_out, H, W, Ho, Wo, K, pad, stride, dil, groups),
                        stream);
}

SOAR_API size_t soar_conv_backward_workspace_bytes(int64_t N, int64_t C_in, int64_t C_out,
                                                   int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                                                   int64_t K, int64_t pad, int64_t stride,
                                                   int64_t dil, int64_t groups) {
    const ConvShape c = conv_shape(N, C_in, C_out, H, W, Ho, Wo, K, pad, stride, dil, groups);
    int64_t ie, oe, we;
    if (check_conv(c, &ie, &oe, &we)) return 0;
    return soar::ops::conv_backward_workspace_bytes(c);
}

SOAR_API int soar_conv_backward(const float* dy, const float* x, const float* weight, float* dx,
                                float* dweight, float* dbias, int64_t N, int64_t C_in,
                                int64_t C_out, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                                int64_t K, int64_t pad, int64_t stride, int64_t dil,
                                int64_t groups, unsigned flags, void* workspace,
                                size_t workspace_bytes, void* stream) {
    if (flags & ~SOAR_GN_ACCUMULATE_DX)
        return fail(SOAR_EINVAL, "conv backward: unknown flags 0x%x", flags);
    return conv_backward(dy, x, weight, dx, dweight, dbias,
                         conv_shape(N, C_in, C_out, H, W, Ho, Wo, K, pad, stride, dil, groups),
                         (flags & SOAR_GN_ACCUMULATE_DX) != 0, workspace, workspace_bytes,
                         stream);
}

// ---- elementwise -------------------------------------------------------------
SOAR_API int soar_sigmoid_forward(const float* x, float* y, size_t n, void* stream) {
    if (n == 0) return ok();
    int rc;
    if ((rc = check_count(n)) || (rc = check_dev(x, n * 4, "x")) || (rc = check_dev(y, n * 4, "y")))
        return rc;
    return launched(soar::ops::launch_sigmoid_forward(x, y, (int64_t)n, S(stream)),
                    "sigmoid_forward launch");
}

SOAR_API int soar_sigmoid_backward_ex(const float* grad_y, const float* y, float* grad_x,
                                      size_t n, unsigned flags, void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "sigmoid_backward", &acc))) return rc;
    if (n == 0) return ok();
    if ((rc = check_count(n)) || (rc = check_dev(grad_y, n * 4, "grad_y")) ||
        (rc = check_dev(y, n * 4, "y")) || (rc = check_dev(grad_x, n * 4, "grad_x")))
        return rc;
    return launched(
        soar::ops::launch_sigmoid_backward(grad_y, y, grad_x, (int64_t)n, acc, S(stream)),
        "sigmoid_backward launch");
}

SOAR_API int soar_sigmoid_backward(const float* grad_y, const float* y, float* grad_x, size_t n,
                                   void* stream) {
    return soar_sigmoid_backward_ex(grad_y, y, grad_x, n, SOAR_GN_ACCUMULATE_DX, stream);
}

SOAR_API int soar_mul_broadcast_forward(const float* a, const float* b, float* y, size_t C,
                                        size_t HW, void* stream) {
    int64_t n;
    int rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (n == 0) return ok();
    if ((rc = require_device()) || (rc = check_dev(a, n * 4, "a")) ||
        (rc = check_dev(b, C * 4, "b")) || (rc = check_dev(y, n * 4, "y")))
        return rc;
    return launched(
        soar::ops::launch_mul_broadcast_forward(a, b, y, (int64_t)C, (int64_t)HW, S(stream)),
        "mul_broadcast_forward launch");
}

SOAR_API int soar_mul_broadcast_backward_ex(const float* grad_y, const float* a,
                                            const float* b, float* grad_a, float* grad_b,
                                            size_t C, size_t HW, unsigned flags, void* stream) {
    int64_t n;
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "mul_broadcast_backward", &acc))) return rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (n == 0 || (!grad_a && !grad_b)) return ok();
    if (C > 0x7fffffffu) return fail(SOAR_EINVAL, "mul_broadcast_backward: C too large");
    if ((rc = require_device()) || (rc = check_dev(grad_y, n * 4, "grad_y")) ||
        (rc = check_dev(a, n * 4, "a")) || (rc = check_dev(b, C * 4, "b")) ||
        (rc = check_dev_opt(grad_a, n * 4, "grad_a")) ||
        (rc = check_dev_opt(grad_b, C * 4, "grad_b")))
        return rc;
    return launched(soar::ops::launch_mul_broadcast_backward(grad_y, a, b, grad_a, grad_b,
                                                             (int64_t)C, (int64_t)HW, acc,
                                                             S(stream)),
                    "mul_broadcast_backward launch");
}

SOAR_API int soar_mul_broadcast_backward(const float* grad_y, const float* a, const float* b,
                                         float* grad_a, float* grad_b, size_t C, size_t HW,
                                         void* stream) {
    return soar_mul_broadcast_backward_ex(grad_y, a, b, grad_a, grad_b, C, HW,
                                          SOAR_GN_ACCUMULATE_DX, stream);
}

SOAR_API int soar_convex_combination_forward(const float* g, const float* a, const float* b,
                                             float* y, size_t n, void* stream) {
    if (n == 0) return ok();
    int rc;
    if ((rc = check_count(n)) || (rc = check_dev(g, n * 4, "g")) ||
        (rc = check_dev(a, n * 4, "a")) || (rc = check_dev(b, n * 4, "b")) ||
        (rc = check_dev(y, n * 4, "y")))
        return rc;
    return launched(soar::ops::launch_convex_forward(g, a, b, y, (int64_t)n, S(stream)),
                    "convex_combination_forward launch");
}

SOAR_API int soar_convex_combination_backward_ex(const float* grad_y, const float* g,
                                                 const float* a, const float* b, float* grad_g,
                                                 float* grad_a, float* grad_b, size_t n,
                                                 unsigned flags, void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "convex_combination_backward", &acc))) return rc;
    if (n == 0 || (!grad_g && !grad_a && !grad_b)) return ok();
    if ((rc = check_count(n)) || (rc = check_dev(grad_y, n * 4, "grad_y")) ||
        (rc = check_dev(g, n * 4, "g")) || (rc = check_dev(a, n * 4, "a")) ||
        (rc = check_dev(b, n * 4, "b")) || (rc = check_dev_opt(grad_g, n * 4, "grad_g")) ||
        (rc = check_dev_opt(grad_a, n * 4, "grad_a")) ||
        (rc = check_dev_opt(grad_b, n * 4, "grad_b")))
        return rc;
    return launched(soar::ops::launch_convex_backward(grad_y, g, a, b, grad_g, grad_a, grad_b,
                                                      (int64_t)n, acc, S(stream)),
                    "convex_combination_backward launch");
}

SOAR_API int soar_convex_combination_backward(const float* grad_y, const float* g,
                                              const float* a, const float* b, float* grad_g,
                                              float* grad_a, float* grad_b, size_t n,
                                              void* stream) {
    return soar_convex_combination_backward_ex(grad_y, g, a, b, grad_g, grad_a, grad_b, n,
                                               SOAR_GN_ACCUMULATE_DX, stream);
}

SOAR_API int soar_sigmoid_convex_forward(const float* z, const float* a, const float* b,
                                         float* y, size_t n, void* stream) {
    if (n == 0) return ok();
    int rc;
    if ((rc = check_count(n)) || (rc = check_dev(z, n * 4, "z")) ||
        (rc = check_dev(a, n * 4, "a")) || (rc = check_dev(b, n * 4, "b")) ||
        (rc = check_dev(y, n * 4, "y")))
        return rc;
    return launched(soar::ops::launch_sigmoid_convex_forward(z, a, b, y, (int64_t)n, S(stream)),
                    "sigmoid_convex_forward launch");
}

SOAR_API int soar_sigmoid_convex_backward_ex(const float* grad_y, const float* z,
                                             const float* a, const float* b, float* grad_z,
                                             float* grad_a, float* grad_b, size_t n,
                                             unsigned flags, void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "sigmoid_convex_backward", &acc))) return rc;
    if (n == 0 || (!grad_z && !grad_a && !grad_b)) return ok();
    if ((rc = check_count(n)) || (rc = check_dev(grad_y, n * 4, "grad_y")) ||
        (rc = check_dev(z, n * 4, "z")) || (rc = check_dev(a, n * 4, "a")) ||
        (rc = check_dev(b, n * 4, "b")) || (rc = check_dev_opt(grad_z, n * 4, "grad_z")) ||
        (rc = check_dev_opt(grad_a, n * 4, "grad_a")) ||
        (rc = check_dev_opt(grad_b, n * 4, "grad_b")))
        return rc;
    return launched(soar::ops::launch_sigmoid_convex_backward(grad_y, z, a, b, grad_z, grad_a,
                                                              grad_b, (int64_t)n, acc,
                                                              S(stream)),
                    "sigmoid_convex_backward launch");
}

SOAR_API int soar_mul_sigmoid_broadcast_forward(const float* a, const float* z, float* y,
                                                size_t C, size_t HW, void* stream) {
    int64_t n;
    int rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (n == 0) return ok();
    if ((rc = require_device()) || (rc = check_dev(a, n * 4, "a")) ||
        (rc = check_dev(z, C * 4, "z")) || (rc = check_dev(y, n * 4, "y")))
        return rc;
    return launched(
        soar::ops::launch_mul_sigmoid_forward(a, z, y, (int64_t)C, (int64_t)HW, S(stream)),
        "mul_sigmoid_broadcast_forward launch");
}

SOAR_API int soar_mul_sigmoid_broadcast_backward_ex(const float* grad_y, const float* a,
                                                    const float* z, float* grad_a,
                                                    float* grad_z, size_t C, size_t HW,
                                                    unsigned flags, void* stream) {
    int64_t n;
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "mul_sigmoid_broadcast_backward", &acc))) return rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (n == 0 || (!grad_a && !grad_z)) return ok();
    if (C > 0x7fffffffu)
        return fail(SOAR_EINVAL, "mul_sigmoid_broadcast_backward: C too large");
    if ((rc = require_device()) || (rc = check_dev(grad_y, n * 4, "grad_y")) ||
        (rc = check_dev(a, n * 4, "a")) || (rc = check_dev(z, C * 4, "z")) ||
        (rc = check_dev_opt(grad_a, n * 4, "grad_a")) ||
        (rc = check_dev_opt(grad_z, C * 4, "grad_z")))
        return rc;
    return launched(soar::ops::launch_mul_sigmoid_backward(grad_y, a, z, grad_a, grad_z,
                                                           (int64_t)C, (int64_t)HW, acc,
                                                           S(stream)),
                    "mul_sigmoid_broadcast_backward launch");
}

SOAR_API int soar_global_avg_pool_forward(const float* in, float* out, size_t C, size_t HW,
                                          void* stream) {
    int64_t n;
    int rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (C == 0) return ok();
    if (HW == 0) return fail(SOAR_EINVAL, "global_avg_pool_forward: empty plane");
    if (C > 0x7fffffffu) return fail(SOAR_EINVAL, "global_avg_pool_forward: C too large");
    if ((rc = require_device()) || (rc = check_dev(in, n * 4, "in")) ||
        (rc = check_dev(out, C * 4, "out")))
        return rc;
    return launched(
        soar::ops::launch_avg_pool_forward(in, out, (int64_t)C, (int64_t)HW, S(stream)),
        "global_avg_pool_forward launch");
}

SOAR_API int soar_global_avg_pool_backward_ex(const float* grad_out, float* grad_in, size_t C,
                                              size_t HW, unsigned flags, void* stream) {
    int64_t n;
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "global_avg_pool_backward", &acc))) return rc;
    if ((rc = check_planes(C, HW, &n))) return rc;
    if (n == 0) return ok();
    if ((rc = require_device()) || (rc = check_dev(grad_out, C * 4, "grad_out")) ||
        (rc = check_dev(grad_in, n * 4, "grad_in")))
        return rc;
    return launched(soar::ops::launch_avg_pool_backward(grad_out, grad_in, (int64_t)C,
                                                        (int64_t)HW, acc, S(stream)),
                    "global_avg_pool_backward launch");
}

SOAR_API int soar_global_avg_pool_backward(const float* grad_out, float* grad_in, size_t C,
                                           size_t HW, void* stream) {
    return soar_global_avg_pool_backward_ex(grad_out, grad_in, C, HW, SOAR_GN_ACCUMULATE_DX,
                                            stream);
}

SOAR_API int soar_upsample_bilinear_forward(const float* in, float* out, size_t C, size_t H_in,
                                            size_t W_in, size_t H_out, size_t W_out,
                                            void* stream) {
    if (C == 0) return ok();
    int rc;
    if ((rc = resize_check(in, out, C, H_in, W_in, H_out, W_out, false))) return rc;
    const int tok = soar::gn::prof_begin(S(stream), "upsample_fwd");
    hipError_t e = soar::ops::launch_upsample_forward(in, out, (int64_t)C, (int64_t)H_in,
                                                      (int64_t)W_in, (int64_t)H_out,
                                                      (int64_t)W_out, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "upsample_bilinear_forward launch");
}

SOAR_API int soar_upsample_bilinear_2x_forward(const float* in, float* out, size_t C,
                                               size_t H_in, size_t W_in, void* stream) {
    if (H_in > (size_t)INT64_MAX / 16 || W_in > (size_t)INT64_MAX / 16)
        return fail(SOAR_EINVAL, "upsample: sizes overflow");
    return soar_upsample_bilinear_forward(in, out, C, H_in, W_in, 2 * H_in, 2 * W_in, stream);
}

SOAR_API int soar_upsample_bilinear_backward_ex(const float* grad_out, float* grad_in,
                                                size_t C, size_t H_in, size_t W_in,
                                                size_t H_out, size_t W_out, unsigned flags,
                                                void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "upsample_bilinear_backward", &acc))) return rc;
    if (C == 0) return ok();
    if ((rc = resize_check(grad_out, grad_in, C, H_in, W_in, H_out, W_out, true))) return rc;
    const int tok = soar::gn::prof_begin(S(stream), "upsample_bwd");
    hipError_t e = soar::ops::launch_upsample_backward(grad_out, grad_in, (int64_t)C,
                                                       (int64_t)H_in, (int64_t)W_in,
                                                       (int64_t)H_out, (int64_t)W_out, acc,
                                                       S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "upsample_bilinear_backward launch");
}

SOAR_API int soar_upsample_bilinear_backward(const float* grad_out, float* grad_in, size_t C,
                                             size_t H_in, size_t W_in, size_t H_out,
                                             size_t W_out, void* stream) {
    return soar_upsample_bilinear_backward_ex(grad_out, grad_in, C, H_in, W_in, H_out, W_out,
                                              SOAR_GN_ACCUMULATE_DX, stream);
}

SOAR_API int soar_upsample_bilinear_2x_backward(const float* grad_out, float* grad_in, size_t C,
                                                size_t H_in, size_t W_in, void* stream) {
    if (H_in > (size_t)INT64_MAX / 16 || W_in > (size_t)INT64_MAX / 16)
        return fail(SOAR_EINVAL, "upsample: sizes overflow");
    return soar_upsample_bilinear_backward(grad_out, grad_in, C, H_in, W_in, 2 * H_in, 2 * W_in,
                                           stream);
}

static int pixel_shuffle(const float* src, float* dst, size_t C_in, size_t H_in, size_t W_in,
                         size_t r, bool backward, bool acc, void* stream) {
    int64_t n;
    if (r == 0 || !fits_i64({C_in, H_in, W_in, r}) ||
        !mul_ok({(int64_t)C_in, (int64_t)H_in, (int64_t)W_in}, &n))
        return fail(SOAR_EINVAL, "pixel_shuffle: invalid sizes");
    if (C_in % (r * r))
        return fail(SOAR_EINVAL, "pixel_shuffle: C_in=%zu is not divisible by r*r=%zu", C_in,
                    r * r);
    if (n == 0) return ok();
    int rc;
    if ((rc = require_device()) || (rc = check_dev(src, n * 4, backward ? "grad_out" : "in")) ||
        (rc = check_dev(dst, n * 4, backward ? "grad_in" : "out")))
        return rc;
    return launched(soar::ops::launch_pixel_shuffle(src, dst, 1, (int64_t)C_in, (int64_t)H_in,
                                                    (int64_t)W_in, (int64_t)r, backward, acc,
                                                    S(stream)),
                    "pixel_shuffle launch");
}

SOAR_API int soar_pixel_shuffle_forward(const float* in, float* out, size_t C_in, size_t H_in,
                                        size_t W_in, size_t r, void* stream) {
    return pixel_shuffle(in, out, C_in, H_in, W_in, r, false, false, stream);
}

SOAR_API int soar_pixel_shuffle_backward_ex(const float* grad_out, float* grad_in, size_t C_in,
                                            size_t H_in, size_t W_in, size_t r, unsigned flags,
                                            void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "pixel_shuffle_backward", &acc))) return rc;
    return pixel_shuffle(grad_out, grad_in, C_in, H_in, W_in, r, true, acc, stream);
}

SOAR_API int soar_pixel_shuffle_backward(const float* grad_out, float* grad_in, size_t C_in,
                                         size_t H_in, size_t W_in, size_t r, void* stream) {
    return soar_pixel_shuffle_backward_ex(grad_out, grad_in, C_in, H_in, W_in, r,
                                          SOAR_GN_ACCUMULATE_DX, stream);
}

static int pad_op(const float* src, float* dst, size_t C, size_t H, size_t W, size_t ph,
                  size_t pw, bool backward, void* stream) {
    int64_t ni, no;
    if (!fits_i64({C, H, W, ph, pw}) || !mul_ok({(int64_t)C, (int64_t)H, (int64_t)W}, &ni) ||
        !mul_ok({(int64_t)C, (int64_t)(H + ph), (int64_t)(W + pw)}, &no))
        return fail(SOAR_EINVAL, "pad_spatial: sizes overflow");
    if (C == 0) return ok();
    if (H == 0 || W == 0) return fail(SOAR_EINVAL, "pad_spatial: empty plane");
    int rc;
    if ((rc = require_device())) return rc;
    if (backward) {
        if ((rc = check_dev(src, no * 4, "grad_out")) || (rc = check_dev(dst, ni * 4, "grad_in")))
            return rc;
    } else if ((rc = check_dev(src, ni * 4, "in")) || (rc = check_dev(dst, no * 4, "out"))) {
        return rc;
    }
    const bool reflect = ph < H && pw < W;  // soar_model.cpp:96
    hipError_t e =
        backward ? soar::ops::launch_pad_backward(src, dst, (int64_t)C, (int64_t)H, (int64_t)W,
                                                  (int64_t)ph, (int64_t)pw, reflect, S(stream))
                 : soar::ops::launch_pad_forward(src, dst, (int64_t)C, (int64_t)H, (int64_t)W,
                                                 (int64_t)ph, (int64_t)pw, reflect, S(stream));
    return launched(e, "pad_spatial launch");
}

SOAR_API int soar_pad_spatial_forward(const float* in, float* out, size_t C, size_t H, size_t W,
                                      size_t ph, size_t pw, void* stream) {
    return pad_op(in, out, C, H, W, ph, pw, false, stream);
}

SOAR_API int soar_pad_spatial_backward(const float* grad_out, float* grad_in, size_t C, size_t H,
                                       size_t W, size_t ph, size_t pw, void* stream) {
    return pad_op(grad_out, grad_in, C, H, W, ph, pw, true, stream);
}

static int crop_op(const float* src, float* dst, size_t C, size_t Hp, size_t Wp, size_t H,
                   size_t W, bool backward, void* stream) {
    int64_t np, nc;
    if (!fits_i64({C, Hp, Wp, H, W}) || !mul_ok({(int64_t)C, (int64_t)Hp, (int64_t)Wp}, &np) ||
        !mul_ok({(int64_t)C, (int64_t)H, (int64_t)W}, &nc))
        return fail(SOAR_EINVAL, "unpad_spatial: sizes overflow");
    if (H > Hp || W > Wp)
        return fail(SOAR_EINVAL, "unpad_spatial: crop %zux%zu exceeds the padded %zux%zu", H, W,
                    Hp, Wp);
    if (nc == 0) return ok();
    int rc;
    if ((rc = require_device())) return rc;
    if (backward) {
        if ((rc = check_dev(src, nc * 4, "grad_out")) || (rc = check_dev(dst, np * 4, "grad_in")))
            return rc;
    } else if ((rc = check_dev(src, np * 4, "in")) || (rc = check_dev(dst, nc * 4, "out"))) {
        return rc;
    }
    return launched(soar::ops::launch_crop(src, dst, (int64_t)C, (int64_t)Hp, (int64_t)Wp,
                                           (int64_t)H, (int64_t)W, backward, S(stream)),
                    "unpad_spatial launch");
}

SOAR_API int soar_unpad_spatial_forward(const float* in, float* out, size_t C, size_t H_pad,
                                        size_t W_pad, size_t H, size_t W, void* stream) {
    return crop_op(in, out, C, H_pad, W_pad, H, W, false, stream);
}

SOAR_API int soar_unpad_spatial_backward(const float* grad_out, float* grad_in, size_t C,
                                         size_t H_pad, size_t W_pad, size_t H, size_t W,
                                         void* stream) {
    return crop_op(grad_out, grad_in, C, H_pad, W_pad, H, W, true, stream);
}

// ---- losses -------------------------------------------------------------------
SOAR_API int soar_bce_with_logits_forward(const float* logits, const float* targets,
                                          float weight, float pos_weight, size_t n,
                                          float* out_loss, void* stream) {
    if (!out_loss) return fail(SOAR_EINVAL, "out_loss is NULL");
    if (n == 0) {
        *out_loss = 0.0f;
        return ok();
    }
    double s[4];
    int rc;
    if ((rc = loss_sums(logits, targets, n, pos_weight, s, stream))) return rc;
    *out_loss = (float)(weight * (s[0] / (double)n));
    return ok();
}

SOAR_API int soar_bce_with_logits_backward(const float* logits, const float* targets,
                                           float* grad_logits, float grad_out, float weight,
                                           float pos_weight, size_t n, void* stream) {
    return loss_bwd(logits, targets, grad_logits, n, grad_out, weight, 1.0f, 0.0f, pos_weight,
                    1.0f, 0.0f, 0.0f, 0.0f, stream);
}

SOAR_API int soar_dice_loss_forward(const float* logits, const float* targets, float weight,
                                    float smooth, float* out_inter, float* out_sum_p,
                                    float* out_sum_y, size_t n, float* out_loss, void* stream) {
    if (!out_loss || !out_inter || !out_sum_p || !out_sum_y)
        return fail(SOAR_EINVAL, "dice_loss_forward: a host output pointer is NULL");
    if (n == 0) {
        *out_loss = *out_inter = *out_sum_p = *out_sum_y = 0.0f;
        return ok();
    }
    double s[4];
    int rc;
    if ((rc = loss_sums(logits, targets, n, 1.0f, s, stream))) return rc;
    float bce, dice;
    finish_losses(s, n, 1.0f, smooth, &bce, &dice, out_inter, out_sum_p, out_sum_y);
    *out_loss = weight * dice;
    return ok();
}

SOAR_API int soar_dice_loss_backward(const float* logits, const float* targets,
                                     float* grad_logits, float grad_out, float weight,
                                     float smooth, float inter, float sum_p, float sum_y,
                                     size_t n, void* stream) {
    return loss_bwd(logits, targets, grad_logits, n, grad_out, weight, 0.0f, 1.0f, 1.0f, smooth,
                    inter, sum_p, sum_y, stream);
}

SOAR_API int soar_dice_bce_loss_forward(const float* logits, const float* targets, size_t n,
                                        float weight, float bce_weight, float dice_weight,
                                        float pos_weight, float smooth, float* out,
                                        void* stream) {
    if (!out) return fail(SOAR_EINVAL, "out is NULL");
    if (n == 0) {
        for (int k = 0; k < 6; ++k) out[k] = 0.0f;
        return ok();
    }
    double s[4];
    int rc;
    if ((rc = loss_sums(logits, targets, n, pos_weight, s, stream))) return rc;
    float bce, dice;
    finish_losses(s, n, pos_weight, smooth, &bce, &dice, &out[3], &out[4], &out[5]);
    out[0] = weight * (bce_weight * bce + dice_weight * dice);  // losses.cpp:477
    out[1] = bce;
    out[2] = dice;
    return ok();
}

SOAR_API int soar_dice_bce_loss_backward_ex(const float* logits, const float* targets,
                                            float* grad_logits, float grad_out, float w, float bw,
                                            float dw, float pos_weight, float smooth, float inter,
                                            float sum_p, float sum_y, size_t n, unsigned flags,
                                            void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "dice_bce_loss_backward", &acc))) return rc;
    return loss_bwd(logits, targets, grad_logits, n, grad_out, w, bw, dw, pos_weight, smooth,
                    inter, sum_p, sum_y, stream, acc);
}

SOAR_API size_t soar_dice_bce_loss_workspace_bytes(size_t n) {
    return n == 0 ? 0 : soar::ops::loss_sums_workspace_bytes((int64_t)n);
}

SOAR_API int soar_dice_bce_loss_sums_device(const float* logits, const float* targets, size_t n,
                                            float pos_weight, double* sums, void* workspace,
                                            size_t workspace_bytes, void* stream) {
    int rc;
    if ((rc = require_device()) || (rc = check_dev(sums, 4 * sizeof(double), "sums"))) return rc;
    if (n == 0) return ok();  // (the caller's finish treats n == 0 itself)
    if ((rc = check_count(n)) || (rc = check_dev(logits, n * 4, "logits")) ||
        (rc = check_dev(targets, n * 4, "targets")))
        return rc;
    const size_t need = soar::ops::loss_sums_workspace_bytes((int64_t)n);
    if (workspace_bytes < need)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu needed",
                    workspace_bytes, need);
    if ((rc = check_dev(workspace, need, "workspace"))) return rc;
    const int tok = soar::gn::prof_begin(S(stream), "dice_bce_sums");
    hipError_t e = soar::ops::launch_loss_sums(logits, targets, (int64_t)n, pos_weight, sums,
                                               workspace, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "loss sums launch");
}

SOAR_API int soar_dice_bce_loss_from_sums(const double* sums, size_t n, float weight,
                                          float bce_weight, float dice_weight, float smooth,
                                          float* out) {
    if (!out || (n > 0 && !sums)) return fail(SOAR_EINVAL, "sums and out must not be NULL");
    if (n == 0) {
        for (int k = 0; k < 6; ++k) out[k] = 0.0f;
        return ok();
    }
    float bce, dice;
    finish_losses(sums, n, 1.0f, smooth, &bce, &dice, &out[3], &out[4], &out[5]);
    out[0] = weight * (bce_weight * bce + dice_weight * dice);  // losses.cpp:477
    out[1] = bce;
    out[2] = dice;
    return ok();
}

SOAR_API int soar_dice_bce_loss_backward_device(const float* logits, const float* targets,
                                                float* grad_logits, float grad_out, float w,
                                                float bw, float dw, float pos_weight,
                                                float smooth, const double* sums, size_t n,
                                                unsigned flags, void* stream) {
    bool acc;
    int rc;
    if ((rc = grad_flags(flags, "dice_bce_loss_backward_device", &acc))) return rc;
    if (n == 0) return ok();
    if ((rc = require_device()) || (rc = check_count(n)) ||
        (rc = check_dev(sums, 4 * sizeof(double), "sums")) ||
        (rc = check_dev(logits, n * 4, "logits")) || (rc = check_dev(targets, n * 4, "targets")) ||
        (rc = check_dev(grad_logits, n * 4, "grad_logits")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "dice_bce_bwd");
    hipError_t e = soar::ops::launch_dice_bce_backward(logits, targets, grad_logits, (int64_t)n,
                                                       grad_out, w, bw, dw, pos_weight, smooth,
                                                       0.0f, 0.0f, 0.0f, acc, S(stream), sums);
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "loss backward launch");
}

SOAR_API int soar_dice_bce_loss_backward(const float* logits, const float* targets,
                                         float* grad_logits, float grad_out, float w, float bw,
                                         float dw, float pos_weight, float smooth, float inter,
                                         float sum_p, float sum_y, size_t n, void* stream) {
    return soar_dice_bce_loss_backward_ex(logits, targets, grad_logits, grad_out, w, bw, dw,
                                          pos_weight, smooth, inter, sum_p, sum_y, n,
                                          SOAR_GN_ACCUMULATE_DX, stream);
}

SOAR_API int soar_sigmoid_threshold(const float* logits, float* probs, uint8_t* mask, size_t n,
                                    float threshold, void* stream) {
    if (n == 0 || (!probs && !mask)) return ok();
    int rc;
    if ((rc = check_count(n)) || (rc = check_dev(logits, n * 4, "logits")) ||
        (rc = check_dev_opt(probs, n * 4, "probs")) || (rc = check_dev_opt(mask, n, "mask")))
        return rc;
    return launched(soar::ops::launch_sigmoid_threshold(logits, probs, mask, (int64_t)n,
                                                        threshold, S(stream)),
                    "sigmoid_threshold launch");
}

// ---- AdamW / multi-tensor -------------------------------------------------------
SOAR_API int soar_adamw_step(float* theta, const float* g, float* m, float* v, float lr,
                             float beta1, float beta2, float eps, float wd, float step_size,
                             float sqrt_bc2, size_t n, void* stream) {
    if (n == 0) return ok();
    int rc;
    if ((rc = check_count(n)) || (rc = check_dev(theta, n * 4, "theta")) ||
        (rc = check_dev(g, n * 4, "g")) || (rc = check_dev(m, n * 4, "m")) ||
        (rc = check_dev(v, n * 4, "v")))
        return rc;
    // a one-entry table in the library's buffer
    void* buf = nullptr;
    if ((rc = table_buffer(5 * 8, &buf))) return rc;
    hipError_t e = hipStreamSynchronize(S(stream));
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    const int64_t nn = (int64_t)n;
    const void* host[5] = {theta, g, m, v, nullptr};
    std::memcpy(&host[4], &nn, 8);
    e = hipMemcpy(buf, host, sizeof host, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "tensor table upload");
    void* const* t = static_cast<void* const*>(buf);
    return launched(soar::ops::launch_adamw_multi(
                        (float* const*)&t[0], (const float* const*)&t[1], (float* const*)&t[2],
                        (float* const*)&t[3], (const int64_t*)&t[4], 1, lr, beta1, beta2, eps,
                        wd, step_size, sqrt_bc2, S(stream)),
                    "adamw_step launch");
}

SOAR_API int soar_adamw_step_multi_tensor(float** params, const float** grads, float** m,
                                          float** v, const int64_t* numel, int n_tensors,
                                          float lr, float beta1, float beta2, float eps, float wd,
                                          float step_size, float sqrt_bc2, void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0 || n_tensors > soar::ops::kMaxMultiTensors || !params || !grads || !m ||
        !v || !numel)
        return fail(SOAR_EINVAL, "adamw_step_multi_tensor: bad table (at most %d tensors)",
                    soar::ops::kMaxMultiTensors);
    int rc;
    if ((rc = require_device())) return rc;
    for (int k = 0; k < n_tensors; ++k) {
        if (numel[k] < 0 || numel[k] > ((int64_t)1 << 42))
            return fail(SOAR_EINVAL, "adamw_step_multi_tensor: numel[%d] is invalid", k);
        if (numel[k] == 0) continue;
        const size_t b = (size_t)numel[k] * 4;
        if ((rc = check_dev(params[k], b, "params[k]")) || (rc = check_dev(grads[k], b, "grads[k]")) ||
            (rc = check_dev(m[k], b, "m[k]")) || (rc = check_dev(v[k], b, "v[k]")))
            return fail(rc, "adamw_step_multi_tensor: tensor %d: %s", k, g_err.c_str());
    }
    int64_t chunks = 0;
    for (int k = 0; k < n_tensors; ++k) chunks += (numel[k] + 4095) / 4096;
    if (chunks >= ((int64_t)1 << 31))
        return fail(SOAR_EINVAL, "adamw_step_multi_tensor: too many elements for one launch");
    const size_t nb = (size_t)n_tensors * 8;
    void* buf = nullptr;
    if ((rc = table_buffer(5 * nb, &buf))) return rc;
    hipError_t e = hipStreamSynchronize(S(stream));  // the previous table is no longer read
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    std::vector<unsigned char> host(5 * nb);
    std::memcpy(host.data(), params, nb);
    std::memcpy(host.data() + nb, grads, nb);
    std::memcpy(host.data() + 2 * nb, m, nb);
    std::memcpy(host.data() + 3 * nb, v, nb);
    std::memcpy(host.data() + 4 * nb, numel, nb);
    e = hipMemcpy(buf, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "tensor table upload");
    unsigned char* d = static_cast<unsigned char*>(buf);
    return launched(soar::ops::launch_adamw_multi(
                        (float* const*)d, (const float* const*)(d + nb), (float* const*)(d + 2 * nb),
                        (float* const*)(d + 3 * nb), (const int64_t*)(d + 4 * nb), n_tensors, lr,
                        beta1, beta2, eps, wd, step_size, sqrt_bc2, S(stream)),
                    "adamw_step_multi_tensor launch");
}

SOAR_API int soar_adamw_multi_tensor_device(float* const* params, const float* const* grads,
                                            float* const* m, float* const* v,
                                            const int64_t* numel, int n_tensors, float lr,
                                            float beta1, float beta2, float eps, float wd,
                                            float step_size, float sqrt_bc2, void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_table(params, n_tensors, "params")) ||
        (rc = check_table(grads, n_tensors, "grads")) || (rc = check_table(m, n_tensors, "m")) ||
        (rc = check_table(v, n_tensors, "v")) || (rc = check_table(numel, n_tensors, "numel")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "adamw_multi");
    hipError_t e = soar::ops::launch_adamw_multi(params, grads, m, v, numel, n_tensors, lr, beta1,
                                                 beta2, eps, wd, step_size, sqrt_bc2, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "adamw multi-tensor launch");
}

SOAR_API int soar_adamw_multi_tensor_device_scalars(
    float* const* params, const float* const* grads, float* const* m, float* const* v,
    const int64_t* numel, int n_tensors, const float* scalars, float beta1, float beta2,
    float eps, float wd, void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_dev(scalars, 3 * sizeof(float), "scalars")) ||
        (rc = check_table(params, n_tensors, "params")) ||
        (rc = check_table(grads, n_tensors, "grads")) || (rc = check_table(m, n_tensors, "m")) ||
        (rc = check_table(v, n_tensors, "v")) || (rc = check_table(numel, n_tensors, "numel")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "adamw_multi");
    hipError_t e = soar::ops::launch_adamw_multi(params, grads, m, v, numel, n_tensors, 0.0f,
                                                 beta1, beta2, eps, wd, 0.0f, 1.0f, S(stream),
                                                 scalars);
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "adamw multi-tensor launch");
}

SOAR_API int soar_multi_tensor_clip_device(float* const* tensors, const int64_t* numel,
                                           int n_tensors, const double* norm_sq, float max_norm,
                                           void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_dev(norm_sq, sizeof(double), "norm_sq")) ||
        (rc = check_table(tensors, n_tensors, "tensors")) ||
        (rc = check_table(numel, n_tensors, "numel")))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "grad_clip");
    hipError_t e =
        soar::ops::launch_multi_clip(tensors, numel, n_tensors, norm_sq, max_norm, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "multi-tensor clip launch");
}

SOAR_API int soar_multi_tensor_norm_sq_partials_device(const float* const* tensors,
                                                       const int64_t* numel, int n_tensors,
                                                       void* workspace, size_t workspace_bytes,
                                                       void* stream) {
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device())) return rc;
    if (n_tensors > 0 &&
        ((rc = check_table(tensors, n_tensors, "tensors")) ||
         (rc = check_table(numel, n_tensors, "numel"))))
        return rc;
    const size_t need = soar::ops::multi_norm_workspace_bytes();
    if (workspace_bytes < need)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu needed",
                    workspace_bytes, need);
    if ((rc = check_dev(workspace, need, "workspace"))) return rc;
    const int tok = soar::gn::prof_begin(S(stream), "grad_norm");
    hipError_t e = soar::ops::launch_multi_norm_partials(tensors, numel, n_tensors, workspace,
                                                         S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "multi-tensor norm launch");
}

SOAR_API int soar_adamw_clip_multi_tensor_device(
    float* const* params, float* const* grads, float* const* m, float* const* v,
    const int64_t* numel, int n_tensors, const float* scalars, float beta1, float beta2,
    float eps, float wd, const void* norm_workspace, size_t norm_workspace_bytes,
    float max_norm, double* norm_sq, unsigned flags, void* stream) {
    if (flags & ~SOAR_ADAMW_ZERO_GRAD)
        return fail(SOAR_EINVAL, "unsupported flags 0x%x (SOAR_ADAMW_ZERO_GRAD)", flags);
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_dev(norm_sq, sizeof(double), "norm_sq")) ||
        (rc = check_dev(scalars, 3 * sizeof(float), "scalars")))
        return rc;
    const size_t need = soar::ops::multi_norm_workspace_bytes();
    if (norm_workspace_bytes < need)
        return fail(SOAR_EINVAL, "norm workspace of %zu bytes is smaller than the %zu needed",
                    norm_workspace_bytes, need);
    if ((rc = check_dev(norm_workspace, need, "norm_workspace"))) return rc;
    if (n_tensors > 0 &&
        ((rc = check_table(params, n_tensors, "params")) ||
         (rc = check_table(grads, n_tensors, "grads")) || (rc = check_table(m, n_tensors, "m")) ||
         (rc = check_table(v, n_tensors, "v")) || (rc = check_table(numel, n_tensors, "numel"))))
        return rc;
    const int tok = soar::gn::prof_begin(S(stream), "adamw_clip_multi");
    hipError_t e = soar::ops::launch_adamw_clip_multi(
        params, grads, m, v, numel, n_tensors, beta1, beta2, eps, wd, scalars, norm_workspace,
        norm_sq, max_norm, (flags & SOAR_ADAMW_ZERO_GRAD) != 0, S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "clip + AdamW multi-tensor launch");
}

SOAR_API size_t soar_multi_tensor_norm_workspace_bytes(void) {
    return soar::ops::multi_norm_workspace_bytes();
}

SOAR_API int soar_multi_tensor_norm_sq_device(const float* const* tensors, const int64_t* numel,
                                              int n_tensors, double* out, void* workspace,
                                              size_t workspace_bytes, void* stream) {
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_dev(out, 8, "out"))) return rc;
    if (n_tensors > 0 &&
        ((rc = check_table(tensors, n_tensors, "tensors")) ||
         (rc = check_table(numel, n_tensors, "numel"))))
        return rc;
    const size_t need = soar::ops::multi_norm_workspace_bytes();
    if (workspace_bytes < need)
        return fail(SOAR_EINVAL, "workspace of %zu bytes is smaller than the %zu needed",
                    workspace_bytes, need);
    if ((rc = check_dev(workspace, need, "workspace"))) return rc;
    const int tok = soar::gn::prof_begin(S(stream), "grad_norm");
    hipError_t e = soar::ops::launch_multi_norm_sq(tensors, numel, n_tensors, out, workspace,
                                                   S(stream));
    soar::gn::prof_end(S(stream), tok);
    return launched(e, "multi-tensor norm launch");
}

SOAR_API int soar_multi_tensor_scale_device(float* const* tensors, const int64_t* numel,
                                            int n_tensors, float scale, void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_table(tensors, n_tensors, "tensors")) ||
        (rc = check_table(numel, n_tensors, "numel")))
        return rc;
    return launched(soar::ops::launch_multi_scale(tensors, numel, n_tensors, scale, S(stream)),
                    "multi-tensor scale launch");
}

SOAR_API int soar_multi_tensor_fill_device(float* const* tensors, const int64_t* numel,
                                           int n_tensors, float value, void* stream) {
    if (n_tensors == 0) return ok();
    if (n_tensors < 0) return fail(SOAR_EINVAL, "n_tensors is negative");
    int rc;
    if ((rc = require_device()) || (rc = check_table(tensors, n_tensors, "tensors")) ||
        (rc = check_table(numel, n_tensors, "numel")))
        return rc;
    return launched(soar::ops::launch_multi_fill(tensors, numel, n_tensors, value, S(stream)),
                    "multi-tensor fill launch");
}

// ---- channel concatenation ------------------------------------------------------
static int concat_args(const int64_t* channels, int K, int64_t N, int64_t HW,
                       soar::ops::CatArgs* a, int64_t* total) {
    if (K < 1 || K > soar::ops::kMaxCat)
        return fail(SOAR_EINVAL, "concat: K=%d is outside [1, %d]", K, soar::ops::kMaxCat);
    if (!channels) return fail(SOAR_EINVAL, "concat: channels is NULL");
    if (N < 0 || HW < 0) return fail(SOAR_EINVAL, "concat: negative N or HW");
    a->K = K;
    a->c_off[0] = 0;
    for (int k = 0; k < K; ++k) {
        if (channels[k] < 0 ||
            __builtin_add_overflow(a->c_off[k], channels[k], &a->c_off[k + 1]))
            return fail(SOAR_EINVAL, "concat: invalid channel count %lld of piece %d",
                        (long long)channels[k], k);
    }
    if (!mul_ok({N, a->c_off[K], HW}, total)) return fail(SOAR_EINVAL, "concat: sizes overflow");
    return SOAR_OK;
}

SOAR_API int soar_concat_channels_forward(const float* const* srcs, const int64_t* channels,
                                          int K, float* dst, int64_t N, int64_t HW,
                                          void* stream) {
    soar::ops::CatArgs a{};
    int64_t total;
    int rc;
    if ((rc = concat_args(channels, K, N, HW, &a, &total))) return rc;
    if (!srcs) return fail(SOAR_EINVAL, "concat: srcs is NULL");
    if (total == 0) return ok();
    if ((rc = require_device()) || (rc = check_dev(dst, (size_t)total * 4, "dst"))) return rc;
    for (int k = 0; k < K; ++k) {
        const int64_t e = N * channels[k] * HW;
        if (e > 0 && (rc = check_dev(srcs[k], (size_t)e * 4, "srcs[k]"))) return rc;
        a.piece[k] = const_cast<float*>(srcs[k]);
    }
    return launched(soar::ops::launch_concat(a, dst, nullptr, N, HW, false, S(stream)),
                    "concat_channels_forward launch");
}

SOAR_API int soar_concat_channels_backward(const float* grad_dst, float* const* grads,
                                           const int64_t* channels, const unsigned* flags,
                                           int K, int64_t N, int64_t HW, void* stream) {
    soar::ops::CatArgs a{};
    int64_t total;
    int rc;
    if ((rc = concat_args(channels, K, N, HW, &a, &total))) return rc;
    if (!grads) return fail(SOAR_EINVAL, "concat: grads is NULL");
    for (int k = 0; flags && k < K; ++k) {
        if (flags[k] & ~SOAR_GN_ACCUMULATE_DX)
            return fail(SOAR_EINVAL,
                        "concat: unsupported flags 0x%x of piece %d (SOAR_GN_ACCUMULATE_DX only)",
                        flags[k], k);
        if (flags[k] & SOAR_GN_ACCUMULATE_DX) a.acc_mask |= 1u << k;
    }
    if (total == 0) return ok();
    if ((rc = require_device()) || (rc = check_dev(grad_dst, (size_t)total * 4, "grad_dst")))
        return rc;
    for (int k = 0; k < K; ++k) {
        const int64_t e = N * channels[k] * HW;
        if (e > 0 && (rc = check_dev_opt(grads[k], (size_t)e * 4, "grads[k]"))) return rc;
        a.piece[k] = e > 0 ? grads[k] : nullptr;
    }
    return launched(soar::ops::launch_concat(a, nullptr, grad_dst, N, HW, true, S(stream)),
                    "concat_channels_backward launch");
}

}  // extern "C"
