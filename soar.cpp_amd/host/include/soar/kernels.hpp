// kernels.hpp - the reference's host-callable operator API for this path
// (include/soar/cuda/cuda_kernels.hpp:8-20,82-88), same names and argument
// meaning, backed by libsoar_gn.so.  Failures throw soar::DeviceError (the
// reference's no-device stub throws the same, cuda_kernels_stub.cpp:99-110)
// or soar::InvalidArgument for a rejected argument.
#pragma once

#include <cstddef>

#include "soar/core.hpp"

namespace soar::hip::kernels {

bool is_cuda_available();

void cuda_zero(float* ptr, size_t n, void* stream = exec::stream());
void cuda_fill(float* ptr, float val, size_t n, void* stream = exec::stream());

void add_forward(const float* a, const float* b, float* y, size_t n, void* stream = exec::stream());
void add_backward(const float* grad_y, float* grad_a, float* grad_b, size_t n,
                  void* stream = exec::stream());

void silu_forward(const float* x, float* y, size_t n, void* stream = exec::stream());
void silu_backward(const float* grad_y, const float* x, float* grad_x, size_t n,
                   void* stream = exec::stream());

void group_norm_forward(const float* in, const float* gamma, const float* beta, float* out,
                        float* saved_mean, float* saved_rstd, size_t num_groups, size_t C,
                        size_t HW, float eps, void* stream = exec::stream());
void group_norm_backward(const float* grad_out, const float* in, const float* gamma,
                         const float* saved_mean, const float* saved_rstd, float* grad_in,
                         float* grad_gamma, float* grad_beta, size_t num_groups, size_t C,
                         size_t HW, void* stream = exec::stream());

// Turns a libsoar_gn status into an exception (used by the host layer).
void check(int status, const char* what);

}  // namespace soar::hip::kernels
