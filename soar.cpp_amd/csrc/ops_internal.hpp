// ops_internal.hpp - launchers of the model operators (model_ops.hip) used
// by the C-ABI in ops_capi.cpp.  Shapes are validated by the caller; every
// launcher only enqueues work on `s` and returns the launch status.
//
// Layout: activations are planes of H*W floats, row-major, one plane per
// (sample, channel): "rows" below is N*C.  Backward launchers add into
// their gradient outputs (the reference's kernels do, e.g.
// activation_kernels.cu:173, binary_ops_kernels.cu:92-169), except the
// convolution's dx, which is written unless accumulate_dx.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace soar::ops {

// General grouped convolution (zero padding, square kernel K, stride S,
// dilation D) on [N][C_in][H][W] -> [N][C_out][Ho][Wo]; weight
// [C_out][C_in/groups][K][K].
struct ConvShape {
    int64_t N, C_in, C_out, H, W, Ho, Wo, K, pad, S, D, groups;
};

hipError_t launch_conv_forward(const float* in, const float* w, const float* bias, float* out,
                               const ConvShape& c, hipStream_t s);
// Workspace of launch_conv_backward (fp64 partial sums of dW and db).
size_t conv_backward_workspace_bytes(const ConvShape& c);
// dx written (or added to when accumulate_dx), dW and db added to.
hipError_t launch_conv_backward(const float* go, const float* in, const float* w, float* gx,
                                float* gw, float* gb, const ConvShape& c, bool accumulate_dx,
                                void* ws, hipStream_t s);

hipError_t launch_sigmoid_forward(const float* x, float* y, int64_t n, hipStream_t s);
// The backward launchers below add into their gradient outputs when `acc`,
// else overwrite them.
hipError_t launch_sigmoid_backward(const float* gy, const float* y, float* gx, int64_t n,
                                   bool acc, hipStream_t s);

hipError_t launch_mul_broadcast_forward(const float* a, const float* b, float* y, int64_t rows,
                                        int64_t HW, hipStream_t s);
hipError_t launch_mul_broadcast_backward(const float* gy, const float* a, const float* b,
                                         float* ga, float* gb, int64_t rows, int64_t HW, bool acc,
                                         hipStream_t s);

// The Fuse / Ctx gates with the sigmoid folded in: s = sigmoid(z) in place
// of the gate g / b above.
hipError_t launch_sigmoid_convex_forward(const float* z, const float* a, const float* b,
                                         float* y, int64_t n, hipStream_t s);
hipError_t launch_sigmoid_convex_backward(const float* gy, const float* z, const float* a,
                                          const float* b, float* gz, float* ga, float* gb,
                                          int64_t n, bool acc, hipStream_t s);
hipError_t launch_mul_sigmoid_forward(const float* a, const float* z, float* y, int64_t rows,
                                      int64_t HW, hipStream_t s);
hipError_t launch_mul_sigmoid_backward(const float* gy, const float* a, const float* z,
                                       float* ga, float* gz, int64_t rows, int64_t HW, bool acc,
                                       hipStream_t s);

hipError_t launch_convex_forward(const float* g, const float* a, const float* b, float* y,
                                 int64_t n, hipStream_t s);
hipError_t launch_convex_backward(const float* gy, const float* g, const float* a,
                                  const float* b, float* gg, float* ga, float* gb, int64_t n,
                                  bool acc, hipStream_t s);

hipError_t launch_avg_pool_forward(const float* in, float* out, int64_t rows, int64_t HW,
                                   hipStream_t s);
hipError_t launch_avg_pool_backward(const float* go, float* gi, int64_t rows, int64_t HW,
                                    bool acc, hipStream_t s);

hipError_t launch_upsample_forward(const float* in, float* out, int64_t rows, int64_t H_in,
                                   int64_t W_in, int64_t H_out, int64_t W_out, hipStream_t s);
hipError_t launch_upsample_backward(const float* go, float* gi, int64_t rows, int64_t H_in,
                                    int64_t W_in, int64_t H_out, int64_t W_out, bool acc,
                                    hipStream_t s);

hipError_t launch_pixel_shuffle(const float* in, float* out, int64_t N, int64_t C_in,
                                int64_t H_in, int64_t W_in, int64_t r, bool backward, bool acc,
                                hipStream_t s);

hipError_t launch_pad_forward(const float* in, float* out, int64_t rows, int64_t H, int64_t W,
                              int64_t ph, int64_t pw, bool reflect, hipStream_t s);
hipError_t launch_pad_backward(const float* go, float* gi, int64_t rows, int64_t H, int64_t W,
                               int64_t ph, int64_t pw, bool reflect, hipStream_t s);
// Crop [rows][Hp][Wp] -> [rows][H][W] (backward: adds the crop's gradient
// into the top-left H x W of each padded plane).
hipError_t launch_crop(const float* in, float* out, int64_t rows, int64_t Hp, int64_t Wp,
                       int64_t H, int64_t W, bool backward, hipStream_t s);

// Dice + BCE loss sums: out[0] = sum of the per-pixel BCE-with-logits
// terms, out[1] = sum p*y, out[2] = sum p, out[3] = sum y (fp64, fixed
// order).  Workspace: loss_sums_workspace_bytes(n).
size_t loss_sums_workspace_bytes(int64_t n);
hipError_t launch_loss_sums(const float* z, const float* y, int64_t n, float pos_weight,
                            double* out, void* ws, hipStream_t s);
// sums (device, nullable): inter, sum_p, sum_y taken from the loss sums
// there (launch_loss_sums' out) instead of the arguments.
hipError_t launch_dice_bce_backward(const float* z, const float* y, float* gz, int64_t n,
                                    float go, float w, float bw, float dw, float pos_weight,
                                    float smooth, float inter, float sum_p, float sum_y, bool acc,
                                    hipStream_t s, const double* sums = nullptr);

// Probabilities and the thresholded mask of a logit map.
hipError_t launch_sigmoid_threshold(const float* z, float* p, uint8_t* mask, int64_t n,
                                    float threshold, hipStream_t s);

// Channel concatenation of K <= kMaxCat pieces [N][C_k][HW] <-> [N][C][HW]
// (C = c_off[K]).  Forward: piece[k] are the sources, `cat` the output.
// Backward: `gcat` is the concatenation's gradient, piece[k] the pieces'
// gradients (null: skipped), added into when bit k of acc_mask is set,
// else written.
constexpr int kMaxCat = 16;
struct CatArgs {
    float* piece[kMaxCat];
    int64_t c_off[kMaxCat + 1];
    unsigned acc_mask;
    int K;
};
hipError_t launch_concat(const CatArgs& a, float* cat, const float* gcat, int64_t N,
                         int64_t HW, bool backward, hipStream_t s);

// Multi-tensor operators over device arrays of tensor pointers and sizes
// (at most kMaxMultiTensors tensors, each under 2^31 * 4096 elements).
constexpr int kMaxMultiTensors = 2048;
size_t multi_norm_workspace_bytes();
hipError_t launch_multi_norm_sq(const float* const* t, const int64_t* numel, int n_tensors,
                                double* out, void* ws, hipStream_t s);
hipError_t launch_multi_scale(float* const* t, const int64_t* numel, int n_tensors, float scale,
                              hipStream_t s);
hipError_t launch_multi_fill(float* const* t, const int64_t* numel, int n_tensors, float value,
                             hipStream_t s);
// scalars (device, nullable): lr, step_size, sqrt_bc2 read there instead.
hipError_t launch_adamw_multi(float* const* p, const float* const* g, float* const* m,
                              float* const* v, const int64_t* numel, int n_tensors, float lr,
                              float beta1, float beta2, float eps, float wd, float step_size,
                              float sqrt_bc2, hipStream_t s, const float* scalars = nullptr);
// Clip by the coefficient formed on the device from norm_sq[0] (see
// k_multi_clip).
// The norm's block partials alone (into the norm workspace), and the
// tail that finishes them: clip + AdamW (scalars on the device) + zero_grad.
hipError_t launch_multi_norm_partials(const float* const* t, const int64_t* numel,
                                      int n_tensors, void* ws, hipStream_t s);
hipError_t launch_adamw_clip_multi(float* const* p, float* const* g, float* const* m,
                                   float* const* v, const int64_t* numel, int n_tensors,
                                   float beta1, float beta2, float eps, float wd,
                                   const float* scalars, const void* norm_ws, double* norm_out,
                                   float max_norm, bool zero_grad, hipStream_t s);
hipError_t launch_multi_clip(float* const* t, const int64_t* numel, int n_tensors,
                             const double* norm_sq, float max_norm, hipStream_t s);

}  // namespace soar::ops
