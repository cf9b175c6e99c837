// The reference's operator API (cuda_kernels.hpp) over libsoar_gn.so.
#include "soar/kernels.hpp"

#include <string>

#include "soar/core.hpp"
#include "soar_gn.h"

namespace soar::hip::kernels {

void check(int status, const char* what) {
    if (status == SOAR_OK) return;
    const std::string msg = std::string(what) + ": " + soar_last_error();
    switch (status) {
        case SOAR_EINVAL: throw InvalidArgument(msg);
        case SOAR_ENOMEM: throw OutOfMemory(msg);
        default: throw DeviceError(msg);
    }
}

bool is_cuda_available() { return soar_is_device_available() != 0; }

void cuda_zero(float* ptr, size_t n, void* stream) { check(soar_zero(ptr, n, stream), "cuda_zero"); }

void cuda_fill(float* ptr, float val, size_t n, void* stream) {
    check(soar_fill(ptr, val, n, stream), "cuda_fill");
}

void add_forward(const float* a, const float* b, float* y, size_t n, void* stream) {
    check(soar_add_forward(a, b, y, n, stream), "add_forward");
}

void add_backward(const float* grad_y, float* grad_a, float* grad_b, size_t n, void* stream) {
    check(soar_add_backward(grad_y, grad_a, grad_b, n, stream), "add_backward");
}

void silu_forward(const float* x, float* y, size_t n, void* stream) {
    check(soar_silu_forward(x, y, n, stream), "silu_forward");
}

void silu_backward(const float* grad_y, const float* x, float* grad_x, size_t n, void* stream) {
    check(soar_silu_backward(grad_y, x, grad_x, n, stream), "silu_backward");
}

void group_norm_forward(const float* in, const float* gamma, const float* beta, float* out,
                        float* saved_mean, float* saved_rstd, size_t num_groups, size_t C,
                        size_t HW, float eps, void* stream) {
    check(soar_group_norm_forward(in, gamma, beta, out, saved_mean, saved_rstd, num_groups, C,
                                  HW, eps, stream),
          "group_norm_forward");
}

void group_norm_backward(const float* grad_out, const float* in, const float* gamma,
                         const float* saved_mean, const float* saved_rstd, float* grad_in,
                         float* grad_gamma, float* grad_beta, size_t num_groups, size_t C,
                         size_t HW, void* stream) {
    check(soar_group_norm_backward(grad_out, in, gamma, saved_mean, saved_rstd, grad_in,
                                   grad_gamma, grad_beta, num_groups, C, HW, stream),
          "group_norm_backward");
}

}  // namespace soar::hip::kernels
