/*
 * soar_ops.h - C-ABI of the MI355X (gfx950) operators the SOAR model needs
 * around the GroupNorm / convolution path (exported by libsoar_gn.so, next
 * to the entry points of soar_gn.h; same status codes, same conventions).
 *
 * Pointers are DEVICE pointers unless stated; `stream` is a hipStream_t
 * passed as void*.  Work is enqueued asynchronously, except the loss
 * forwards and the host-array multi-tensor entry points, which return
 * host values or read host arrays and say so.  Layout is fp32 planes of
 * H*W floats, one per (sample, channel); where an argument is named C, a
 * caller with N samples passes N*C (the operators treat every plane alike).
 *
 * Backward entry points ADD into their gradient outputs, as the
 * reference's kernels do (activation_kernels.cu:173, binary_ops_kernels.cu:
 * 92-169, pooling_kernels.cu:31, upsample_kernels.cu:97-100,195,
 * convolution_kernels.cu:58,236, loss_kernels.cu:95,195,249): pass zeroed
 * buffers for a fresh gradient.  Reductions run in a fixed order (no float
 * atomics), so every result is reproducible run to run.
 *
 * Reference interfaces replaced (pomagrenate/soar.cpp):
 *   include/soar/cuda/cuda_kernels.hpp:23-48,73-79,91-127
 *   src/cuda/ops/{convolution,activation,binary_ops,pooling,upsample,
 *   loss,optimizer}_kernels.cu, src/nn/soar_model.cpp:15-172 (pad/unpad)
 */
#ifndef SOAR_OPS_H
#define SOAR_OPS_H

#include <stddef.h>
#include <stdint.h>

#include "soar_gn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- general grouped convolution ------------------------------------ */

/* out[co][y][x] = bias[co] + sum over the C_in/groups channels of co's
 * group and the K x K taps of weight[co][q][ky][kx] *
 * in[ci][y*stride - pad + ky*dil][x*stride - pad + kx*dil] (zero outside).
 * weight [C_out][C_in/groups][K][K]; bias may be NULL.  One sample.
 * Replaces: conv2d_forward (cuda_kernels.hpp:73-75). */
SOAR_API int soar_conv2d_forward(const float* in, const float* weight,
                                 const float* bias, float* out, size_t C_in,
                                 size_t C_out, size_t H_in, size_t W_in,
                                 size_t H_out, size_t W_out, size_t K,
                                 size_t pad, size_t stride, size_t dil,
                                 size_t groups, void* stream);

/* grad_in, grad_weight, grad_bias += the gradients of conv2d_forward (any
 * may be NULL).  Uses a library-owned workspace.
 * Replaces: conv2d_backward (cuda_kernels.hpp:76-79). */
SOAR_API int soar_conv2d_backward(const float* grad_out, const float* in,
                                  const float* weight, float* grad_in,
                                  float* grad_weight, float* grad_bias,
                                  size_t C_in, size_t C_out, size_t H_in,
                                  size_t W_in, size_t H_out, size_t W_out,
                                  size_t K, size_t pad, size_t stride,
                                  size_t dil, size_t groups, void* stream);

/* Batched forms for N samples [N][C][H][W] with a caller workspace.  The
 * backward writes dx (adds with SOAR_GN_ACCUMULATE_DX) and adds dweight /
 * dbias (summed over the samples).  Workspace: fp64 per-chunk partial sums
 * of dweight / dbias (0 bytes when neither is wanted is still accepted). */
SOAR_API int soar_conv_forward(const float* x, const float* weight,
                               const float* bias, float* y, int64_t N,
                               int64_t C_in, int64_t C_out, int64_t H,
                               int64_t W, int64_t Ho, int64_t Wo, int64_t K,
                               int64_t pad, int64_t stride, int64_t dil,
                               int64_t groups, void* stream);
SOAR_API size_t soar_conv_backward_workspace_bytes(
    int64_t N, int64_t C_in, int64_t C_out, int64_t H, int64_t W, int64_t Ho,
    int64_t Wo, int64_t K, int64_t pad, int64_t stride, int64_t dil,
    int64_t groups);
SOAR_API int soar_conv_backward(const float* dy, const float* x,
                                const float* weight, float* dx,
                                float* dweight, float* dbias, int64_t N,
                                int64_t C_in, int64_t C_out, int64_t H,
                                int64_t W, int64_t Ho, int64_t Wo, int64_t K,
                                int64_t pad, int64_t stride, int64_t dil,
                                int64_t groups, unsigned flags,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/* ---- elementwise and per-plane operators ----------------------------- */

/* y = 1 / (1 + exp(-x)).  Replaces: sigmoid_forward (cuda_kernels.hpp:23). */
SOAR_API int soar_sigmoid_forward(const float* x, float* y, size_t n,
                                  void* stream);
/* grad_x += grad_y * y * (1 - y), y the forward output.
 * Replaces: sigmoid_backward (cuda_kernels.hpp:24). */
SOAR_API int soar_sigmoid_backward(const float* grad_y, const float* y,
                                   float* grad_x, size_t n, void* stream);

/* y[c][i] = a[c][i] * b[c] over C planes of HW.
 * Replaces: mul_broadcast_forward (cuda_kernels.hpp:27). */
SOAR_API int soar_mul_broadcast_forward(const float* a, const float* b,
                                        float* y, size_t C, size_t HW,
                                        void* stream);
/* grad_a += grad_y * b[c];  grad_b[c] += sum_i grad_y * a (either NULL).
 * Replaces: mul_broadcast_backward (cuda_kernels.hpp:28-29). */
SOAR_API int soar_mul_broadcast_backward(const float* grad_y, const float* a,
                                         const float* b, float* grad_a,
                                         float* grad_b, size_t C, size_t HW,
                                         void* stream);

/* y = g*a + (1-g)*b.  Replaces: convex_combination_forward (cuda_kernels.hpp:32). */
SOAR_API int soar_convex_combination_forward(const float* g, const float* a,
                                             const float* b, float* y,
                                             size_t n, void* stream);
/* grad_g += gy*(a-b); grad_a += gy*g; grad_b += gy*(1-g) (any NULL).
 * Replaces: convex_combination_backward (cuda_kernels.hpp:33-34). */
SOAR_API int soar_convex_combination_backward(
    const float* grad_y, const float* g, const float* a, const float* b,
    float* grad_g, float* grad_a, float* grad_b, size_t n, void* stream);

/* The SOAR gates with their sigmoid folded in (no counterpart in the
 * reference, which runs sigmoid_forward and then the gate's kernel: the
 * same values in one launch per direction; the host layer's Fuse and Ctx
 * blocks use them).  s = sigmoid(z) is recomputed from z as
 * soar_sigmoid_forward computes it.
 *   soar_sigmoid_convex_*: y = s*a + (1-s)*b (as soar_convex_combination_*
 *   with g = s); grad_z = grad_y*(a-b) * s*(1-s), grad_a = grad_y*s,
 *   grad_b = grad_y*(1-s) (any NULL).
 *   soar_mul_sigmoid_broadcast_*: y[c][i] = a[c][i] * s[c] (as
 *   soar_mul_broadcast_* with b = s); grad_a = grad_y*s[c], grad_z[c] =
 *   (sum_i grad_y*a) * s[c]*(1-s[c]) (either NULL).
 * flags as the _ex entry points below: SOAR_GN_ACCUMULATE_DX adds into the
 * gradients, 0 writes them. */
SOAR_API int soar_sigmoid_convex_forward(const float* z, const float* a,
                                         const float* b, float* y, size_t n,
                                         void* stream);
SOAR_API int soar_sigmoid_convex_backward_ex(
    const float* grad_y, const float* z, const float* a, const float* b,
    float* grad_z, float* grad_a, float* grad_b, size_t n, unsigned flags,
    void* stream);
SOAR_API int soar_mul_sigmoid_broadcast_forward(const float* a, const float* z,
                                                float* y, size_t C, size_t HW,
                                                void* stream);
SOAR_API int soar_mul_sigmoid_broadcast_backward_ex(
    const float* grad_y, const float* a, const float* z, float* grad_a,
    float* grad_z, size_t C, size_t HW, unsigned flags, void* stream);

/* out[c] = mean of plane c.  Replaces: global_avg_pool_forward (cuda_kernels.hpp:37). */
SOAR_API int soar_global_avg_pool_forward(const float* in, float* out,
                                          size_t C, size_t HW, void* stream);
/* grad_in[c][i] += grad_out[c] / HW.
 * Replaces: global_avg_pool_backward (cuda_kernels.hpp:38). */
SOAR_API int soar_global_avg_pool_backward(const float* grad_out,
                                           float* grad_in, size_t C,
                                           size_t HW, void* stream);

/* Bilinear resize with half-pixel centres and no corner alignment (source
 * coordinate max(0, (d + 0.5) * in/out - 0.5)), the taps of the last row /
 * column clamped.  Replaces: upsample_bilinear_forward (cuda_kernels.hpp:43),
 * upsample_bilinear_2x_forward (:41). */
SOAR_API int soar_upsample_bilinear_forward(const float* in, float* out,
                                            size_t C, size_t H_in,
                                            size_t W_in, size_t H_out,
                                            size_t W_out, void* stream);
SOAR_API int soar_upsample_bilinear_2x_forward(const float* in, float* out,
                                               size_t C, size_t H_in,
                                               size_t W_in, void* stream);
/* grad_in += the adjoint of the resize (a gather: every input pixel sums
 * the output pixels that read it).  Replaces: upsample_bilinear_backward
 * (cuda_kernels.hpp:44), upsample_bilinear_2x_backward (:42). */
SOAR_API int soar_upsample_bilinear_backward(const float* grad_out,
                                             float* grad_in, size_t C,
                                             size_t H_in, size_t W_in,
                                             size_t H_out, size_t W_out,
                                             void* stream);
SOAR_API int soar_upsample_bilinear_2x_backward(const float* grad_out,
                                                float* grad_in, size_t C,
                                                size_t H_in, size_t W_in,
                                                void* stream);

/* out[c][y][x] = in[c*r*r + (y%r)*r + x%r][y/r][x/r], C_in = C_out*r*r.
 * Replaces: pixel_shuffle_forward / _backward (cuda_kernels.hpp:47-48). */
SOAR_API int soar_pixel_shuffle_forward(const float* in, float* out,
                                        size_t C_in, size_t H_in,
                                        size_t W_in, size_t r, void* stream);
SOAR_API int soar_pixel_shuffle_backward(const float* grad_out,
                                         float* grad_in, size_t C_in,
                                         size_t H_in, size_t W_in, size_t r,
                                         void* stream);

/* Pads [C][H][W] to [C][H+ph][W+pw]: extra rows/columns reflect about the
 * last one (2(H-1)-y) when ph < H and pw < W, else repeat the last one.
 * Replaces: pad_spatial / AutoPadNode (soar_model.cpp:15-38,74-135). */
SOAR_API int soar_pad_spatial_forward(const float* in, float* out, size_t C,
                                      size_t H, size_t W, size_t ph,
                                      size_t pw, void* stream);
SOAR_API int soar_pad_spatial_backward(const float* grad_out, float* grad_in,
                                       size_t C, size_t H, size_t W,
                                       size_t ph, size_t pw, void* stream);
/* Crops [C][H_pad][W_pad] to its top-left [C][H][W].
 * Replaces: unpad_spatial / UnpadNode (soar_model.cpp:40-72,137-172). */
SOAR_API int soar_unpad_spatial_forward(const float* in, float* out, size_t C,
                                        size_t H_pad, size_t W_pad, size_t H,
                                        size_t W, void* stream);
SOAR_API int soar_unpad_spatial_backward(const float* grad_out,
                                         float* grad_in, size_t C,
                                         size_t H_pad, size_t W_pad, size_t H,
                                         size_t W, void* stream);

/* ---- losses (forwards synchronise the stream and return host values) -- */

/* *out_loss = weight * mean_i [(1-y) z + (1 + (pos_weight-1) y) *
 * (max(-z,0) + log1p(exp(-|z|)))].  out_loss is a HOST pointer.
 * Replaces: bce_with_logits_forward (cuda_kernels.hpp:91-92). */
SOAR_API int soar_bce_with_logits_forward(const float* logits,
                                          const float* targets, float weight,
                                          float pos_weight, size_t n,
                                          float* out_loss, void* stream);
/* grad_logits += grad_out * weight / n * (sigmoid(z) (1 + (pw-1) y) - pw y).
 * Replaces: bce_with_logits_backward (cuda_kernels.hpp:93-94). */
SOAR_API int soar_bce_with_logits_backward(const float* logits,
                                           const float* targets,
                                           float* grad_logits, float grad_out,
                                           float weight, float pos_weight,
                                           size_t n, void* stream);
/* Soft Dice: with p = sigmoid(z), inter = sum p*y, sum_p, sum_y (HOST
 * outputs, fp32 as the reference returns them), *out_loss = weight *
 * (1 - (2 inter + smooth) / (sum_p + sum_y + smooth + 1e-7)).
 * Replaces: dice_loss_forward (cuda_kernels.hpp:96-98). */
SOAR_API int soar_dice_loss_forward(const float* logits, const float* targets,
                                    float weight, float smooth,
                                    float* out_inter, float* out_sum_p,
                                    float* out_sum_y, size_t n,
                                    float* out_loss, void* stream);
/* Replaces: dice_loss_backward (cuda_kernels.hpp:99-101). */
SOAR_API int soar_dice_loss_backward(const float* logits, const float* targets,
                                     float* grad_logits, float grad_out,
                                     float weight, float smooth, float inter,
                                     float sum_p, float sum_y, size_t n,
                                     void* stream);
/* Both losses from one pass over logits and targets (DiceBCELoss::forward,
 * losses.cpp:464-478): out[6] (HOST) = {total = weight*(bce_weight*bce +
 * dice_weight*dice), bce, dice, inter, sum_p, sum_y}, bce with weight 1
 * and dice with weight 1 as the DiceBCELoss members compute them. */
SOAR_API int soar_dice_bce_loss_forward(const float* logits,
                                        const float* targets, size_t n,
                                        float weight, float bce_weight,
                                        float dice_weight, float pos_weight,
                                        float smooth, float* out,
                                        void* stream);
/* Replaces: dice_bce_loss_backward (cuda_kernels.hpp:103-105). */
SOAR_API int soar_dice_bce_loss_backward(const float* logits,
                                         const float* targets,
                                         float* grad_logits, float grad_out,
                                         float w, float bw, float dw,
                                         float pos_weight, float smooth,
                                         float inter, float sum_p,
                                         float sum_y, size_t n, void* stream);

/* probs = sigmoid(logits) and mask = probs >= threshold (either output may
 * be NULL; mask is uint8 0/1).  The Predictor's loop (predictor.cpp:67-74)
 * on the device. */
SOAR_API int soar_sigmoid_threshold(const float* logits, float* probs,
                                    uint8_t* mask, size_t n, float threshold,
                                    void* stream);

/* ---- AdamW and multi-tensor operators --------------------------------- */

/* One AdamW step over n elements (adamw.cpp:80-104): theta -= lr*wd*theta;
 * m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2; theta -= step_size *
 * m / (sqrt(v)/sqrt_bc2 + eps), each operation rounded to fp32 separately
 * (no fused multiply-add), so it equals a scalar IEEE evaluation bit for
 * bit.  Replaces: adamw_step (cuda_kernels.hpp:108-110). */
SOAR_API int soar_adamw_step(float* theta, const float* g, float* m, float* v,
                             float lr, float beta1, float beta2, float eps,
                             float wd, float step_size, float sqrt_bc2,
                             size_t n, void* stream);
/* The same over n_tensors tensors in one launch.  The five arrays are HOST
 * arrays of device pointers / sizes; every pointer is validated and the
 * table copied to a library-owned device buffer (the call synchronises the
 * stream first, so the buffer is free).
 * Replaces: adamw_step_multi_tensor (cuda_kernels.hpp:113-127). */
SOAR_API int soar_adamw_step_multi_tensor(float** params, const float** grads,
                                          float** m, float** v,
                                          const int64_t* numel, int n_tensors,
                                          float lr, float beta1, float beta2,
                                          float eps, float wd,
                                          float step_size, float sqrt_bc2,
                                          void* stream);

/* Device-table forms for callers that keep the table resident (e.g. the
 * parameter list of a model): the arrays themselves are DEVICE arrays of
 * n_tensors entries (at most 2048 tensors; the summed chunk count of 4096
 * elements must stay below 2^31).  The pointers inside the table are not
 * validated (the table is not read on the host); only the arrays' own
 * extents are.
 * No counterpart in the reference (its optimizer copies a host table per
 * launch, optimizer_kernels.cu:211-240). */
SOAR_API int soar_adamw_multi_tensor_device(
    float* const* params, const float* const* grads, float* const* m,
    float* const* v, const int64_t* numel, int n_tensors, float lr,
    float beta1, float beta2, float eps, float wd, float step_size,
    float sqrt_bc2, void* stream);
/* *out (device double) = sum of squares of every element, fp64, fixed
 * order.  Workspace: soar_multi_tensor_norm_workspace_bytes(). */
SOAR_API size_t soar_multi_tensor_norm_workspace_bytes(void);
SOAR_API int soar_multi_tensor_norm_sq_device(const float* const* tensors,
                                              const int64_t* numel,
                                              int n_tensors, double* out,
                                              void* workspace,
                                              size_t workspace_bytes,
                                              void* stream);
/* tensors[k][i] *= scale (the clip of AdamW::clip_grad_norm,
 * adamw.cpp:44-54). */
SOAR_API int soar_multi_tensor_scale_device(float* const* tensors,
                                            const int64_t* numel,
                                            int n_tensors, float scale,
                                            void* stream);

/* The same AdamW step with lr, step_size and sqrt_bc2 read from a DEVICE
 * array scalars[3] when the kernel runs, so a captured training step can
 * replay with the next step's values (the caller writes them there, e.g.
 * with a captured copy from pinned memory).  Arithmetic as above. */
SOAR_API int soar_adamw_multi_tensor_device_scalars(
    float* const* params, const float* const* grads, float* const* m,
    float* const* v, const int64_t* numel, int n_tensors,
    const float* scalars, float beta1, float beta2, float eps, float wd,
    void* stream);
/* The clip of AdamW::clip_grad_norm (adamw.cpp:44-54) with its decision on
 * the device: total = (float)sqrt(*norm_sq) (norm_sq a DEVICE double, as
 * soar_multi_tensor_norm_sq_device writes it); when total > max_norm and
 * total > 1e-6 every tensor is scaled by max_norm / total, else nothing
 * changes.  No host read-back (capture-safe). */
SOAR_API int soar_multi_tensor_clip_device(float* const* tensors,
                                           const int64_t* numel, int n_tensors,
                                           const double* norm_sq,
                                           float max_norm, void* stream);

/* The device training step's tail in two launches (no counterpart in the
 * reference, whose trainer clips, steps and zeroes the gradients one after
 * another, trainer.cpp:110-220; these give the values of
 * soar_multi_tensor_norm_sq_device, soar_multi_tensor_clip_device,
 * soar_adamw_multi_tensor_device_scalars and, with SOAR_ADAMW_ZERO_GRAD,
 * soar_multi_tensor_fill_device(0) in that order):
 *   soar_multi_tensor_norm_sq_partials_device: the squared norm's block
 *   partials of `tensors` into the workspace (no finish);
 *   soar_adamw_clip_multi_tensor_device: every block adds those partials
 *   (the finish; *norm_sq, a DEVICE double, receives the squared norm),
 *   clips the gradient by max_norm / total when total = (float)
 *   sqrt(norm_sq) > max_norm and > 1e-6, runs the AdamW update with
 *   scalars[3] (DEVICE: lr, step_size, sqrt_bc2) and, with
 *   SOAR_ADAMW_ZERO_GRAD, sets the gradients to zero (else leaves the
 *   clipped ones).  No host read-back (capture-safe). */
#define SOAR_ADAMW_ZERO_GRAD 1u
SOAR_API int soar_multi_tensor_norm_sq_partials_device(
    const float* const* tensors, const int64_t* numel, int n_tensors,
    void* workspace, size_t workspace_bytes, void* stream);
SOAR_API int soar_adamw_clip_multi_tensor_device(
    float* const* params, float* const* grads, float* const* m,
    float* const* v, const int64_t* numel, int n_tensors,
    const float* scalars, float beta1, float beta2, float eps, float wd,
    const void* norm_workspace, size_t norm_workspace_bytes, float max_norm,
    double* norm_sq, unsigned flags, void* stream);

/* tensors[k][i] = value (one launch for a whole gradient list:
 * Module::zero_grad, module.hpp:71-75, without a launch per tensor). */
SOAR_API int soar_multi_tensor_fill_device(float* const* tensors,
                                           const int64_t* numel, int n_tensors,
                                           float value, void* stream);

/* ---- channel concatenation --------------------------------------------- */
/* dst [N][C][HW] = the K pieces srcs[k] [N][channels[k]][HW] one after the
 * other along channels (C = sum of channels), 1 <= K <= 16.  srcs and
 * channels are HOST arrays of device pointers and counts.  One launch for
 * all pieces and samples.
 * Replaces: concat_channels (blocks.cpp), which copies each piece of each
 * sample with its own device copy. */
SOAR_API int soar_concat_channels_forward(const float* const* srcs,
                                          const int64_t* channels, int K,
                                          float* dst, int64_t N, int64_t HW,
                                          void* stream);
/* Its backward: grads[k] [N][channels[k]][HW] receives piece k's slice of
 * grad_dst, written, or added with flags[k] = SOAR_GN_ACCUMULATE_DX (flags
 * may be NULL: all written); a NULL grads[k] is skipped.  grads, channels
 * and flags are HOST arrays.  Replaces: the ConcatNode backward's copies
 * (blocks.cpp). */
SOAR_API int soar_concat_channels_backward(const float* grad_dst,
                                           float* const* grads,
                                           const int64_t* channels,
                                           const unsigned* flags, int K,
                                           int64_t N, int64_t HW, void* stream);

/* ---- backward entry points that may write instead of add -------------- */
/* Each takes the arguments of the entry point of the same name without
 * _ex, plus `flags`: SOAR_GN_ACCUMULATE_DX adds into the gradient outputs
 * (exactly the entry point without _ex), 0 overwrites them, so a caller
 * making a fresh gradient needs no zeroed buffer (one launch and one
 * write pass fewer).  Any other flag bit is SOAR_EINVAL.  No counterpart in
 * the reference (its kernels always add); the host layer's autograd uses
 * them to write a tensor's first gradient and add the later ones. */
SOAR_API int soar_sigmoid_backward_ex(const float* grad_y, const float* y,
                                      float* grad_x, size_t n, unsigned flags,
                                      void* stream);
SOAR_API int soar_mul_broadcast_backward_ex(const float* grad_y,
                                            const float* a, const float* b,
                                            float* grad_a, float* grad_b,
                                            size_t C, size_t HW, unsigned flags,
                                            void* stream);
SOAR_API int soar_convex_combination_backward_ex(
    const float* grad_y, const float* g, const float* a, const float* b,
    float* grad_g, float* grad_a, float* grad_b, size_t n, unsigned flags,
    void* stream);
SOAR_API int soar_global_avg_pool_backward_ex(const float* grad_out,
                                              float* grad_in, size_t C,
                                              size_t HW, unsigned flags,
                                              void* stream);
SOAR_API int soar_upsample_bilinear_backward_ex(const float* grad_out,
                                                float* grad_in, size_t C,
                                                size_t H_in, size_t W_in,
                                                size_t H_out, size_t W_out,
                                                unsigned flags, void* stream);
SOAR_API int soar_pixel_shuffle_backward_ex(const float* grad_out,
                                            float* grad_in, size_t C_in,
                                            size_t H_in, size_t W_in, size_t r,
                                            unsigned flags, void* stream);
SOAR_API int soar_dice_bce_loss_backward_ex(
    const float* logits, const float* targets, float* grad_logits,
    float grad_out, float w, float bw, float dw, float pos_weight,
    float smooth, float inter, float sum_p, float sum_y, size_t n,
    unsigned flags, void* stream);

/* ---- the Dice+BCE loss with its sums kept on the device ------------------ */
/* No counterpart in the reference: the loss of soar_dice_bce_loss_forward
 * split so that no host read-back sits inside a training step (for stream
 * capture).  sums (DEVICE, 4 doubles) = the BCE sum, sum p*y, sum p, sum y
 * (the same fixed-order fp64 sums); workspace from
 * soar_dice_bce_loss_workspace_bytes(n).  soar_dice_bce_loss_from_sums
 * finishes them on the HOST into the out[6] of soar_dice_bce_loss_forward,
 * bit for bit.  The backward reads inter, sum_p and sum_y from the device
 * sums, handed on as fp32 as the host finish does. */
SOAR_API size_t soar_dice_bce_loss_workspace_bytes(size_t n);
SOAR_API int soar_dice_bce_loss_sums_device(const float* logits,
                                            const float* targets, size_t n,
                                            float pos_weight, double* sums,
                                            void* workspace,
                                            size_t workspace_bytes,
                                            void* stream);
SOAR_API int soar_dice_bce_loss_from_sums(const double* sums, size_t n,
                                          float weight, float bce_weight,
                                          float dice_weight, float smooth,
                                          float* out);
SOAR_API int soar_dice_bce_loss_backward_device(
    const float* logits, const float* targets, float* grad_logits,
    float grad_out, float w, float bw, float dw, float pos_weight,
    float smooth, const double* sums, size_t n, unsigned flags,
    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOAR_OPS_H */
