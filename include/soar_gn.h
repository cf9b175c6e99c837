/*
 * soar_gn.h - C-ABI of the MI355X (gfx950) GroupNorm+SiLU path.
 *
 * One shared library, libsoar_gn.so, exports every function below with
 * C linkage, plain pointers and sizes.  Pointers named x, y, dy, dx, gamma,
 * beta, mean, rstd, dgamma, dbeta, workspace are DEVICE pointers (HBM);
 * `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 * kernels are enqueued asynchronously on that stream; no entry point
 * synchronises the device except where stated.
 *
 * Layout: fp32, NCHW contiguous.  G groups split C channels into runs of
 * C/G consecutive channels; a "unit" (n, g) is the M = (C/G)*H*W contiguous
 * floats those channels occupy in sample n.  mean and rstd are float[N*G]
 * indexed n*G + g.
 *
 * Every entry point returns an int status: SOAR_OK (0) or a negative code,
 * and records a message retrievable with soar_last_error() on the calling
 * thread.  Nothing is launched when a call returns an error.
 *
 * Reference interfaces replaced (pomagrenate/soar.cpp):
 *   include/soar/cuda/cuda_kernels.hpp:8-20,82-88   operator API nn calls
 *   src/cuda/ops/normalization_kernels.cu:93-289     GN forward/backward
 *   src/cuda/ops/activation_kernels.cu:99-130        SiLU forward/backward
 *   src/cuda/ops/binary_ops_kernels.cu:6-102         zero/fill/add
 *   shaders/group_norm_stats.comp, group_norm_affine_silu.comp,
 *   shaders/tensor_add.comp                          Vulkan GN+SiLU pair
 *   src/memory/device_slab.cpp:6-56, src/vulkan/buffer.cpp:8-75,
 *   src/cuda/cuda_allocator.cpp:24-77                device buffers
 */
#ifndef SOAR_GN_H
#define SOAR_GN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SOAR_API __attribute__((visibility("default")))

/* ---- status codes --------------------------------------------------- */
#define SOAR_OK 0
#define SOAR_EINVAL (-1) /* bad pointer, shape, flag or workspace size     */
#define SOAR_ENOMEM (-2) /* device or arena allocation failed              */
#define SOAR_EHIP (-3)   /* a HIP runtime call or kernel launch failed     */
#define SOAR_ENODEV (-4) /* no HIP device visible                          */

/* ---- flags for the fused entry points -------------------------------- */
#define SOAR_GN_SILU 1u          /* apply SiLU after the affine GroupNorm     */
#define SOAR_GN_RESIDUAL 2u      /* fwd: y += x;  bwd: dx += dy (x + f(x))    */
#define SOAR_GN_ACCUMULATE_DX 4u /* bwd: dx += result instead of dx = result  */
/* Convolution backward calls (soar_pw_conv_backward, soar_pw_cba_backward,
 * soar_dw_conv_backward, soar_dw_cba_backward): leave the weight / bias
 * gradient's final addition pending.  The per-block partial sums stay in
 * the call's workspace and dweight / dbias receive them at the next
 * soar_weight_grad_flush on this thread, added exactly as the call itself
 * would have added them (the same float64 sums in the same order), so the
 * gradients are bit for bit the same.  The caller keeps the workspace and
 * the gradient buffers untouched until the flush.  dx is written at once. */
#define SOAR_DEFER_WEIGHT_FINISH 8u

/* Message for the last failing call on this thread ("" if none). */
SOAR_API const char* soar_last_error(void);

/* 1 if a HIP device is visible, else 0.
 * Replaces: soar::cuda::kernels::is_cuda_available (cuda_kernels.hpp:8). */
SOAR_API int soar_is_device_available(void);

/* ---- fused GroupNorm(+SiLU) ------------------------------------------- */

/* Bytes of device workspace the fused entry points need for this shape
 * (0 for an empty tensor).  The workspace holds per-chunk partial moments
 * and sums, per-plane and per-unit sums and the per-unit mean residuals; it
 * carries nothing between calls, and two calls that overlap in time on the
 * device must not share one. */
SOAR_API size_t soar_gn_workspace_bytes(int64_t N, int64_t C, int64_t HW,
                                        int64_t G);

/* Forward: per unit mean and rstd = 1/sqrt(var + eps) (biased variance),
 * then y = f(gamma_c*(x - mean)*rstd + beta_c) [+ x], f = SiLU when
 * SOAR_GN_SILU is set, identity otherwise.  gamma/beta may be NULL (1 / 0,
 * the affine=false module).  y must not overlap x.  Writes mean/rstd (fp32,
 * as the reference saves them) for the backward, and, when mean_lo is not
 * NULL, mean_lo[u] = exact mean - mean[u]: the fp32 rounding residual of
 * the mean.  Passing mean_lo back to the backward keeps xhat exact to fp32
 * rounding even when std << |mean| (e.g. x = 1e3 + N(0, 1e-2)), where the
 * rounded mean alone shifts xhat by up to ulp(mean)/2 * rstd.  The forward
 * output y always uses the exact mean.
 * Replaces: group_norm_forward (cuda_kernels.hpp:82-84) followed by
 * silu_forward (:19), the Vulkan pair group_norm_stats.comp +
 * group_norm_affine_silu.comp, and with SOAR_GN_RESIDUAL the add_forward
 * (:15) of a residual block (src/nn/blocks.cpp:478-480). */
SOAR_API int soar_gn_silu_forward(const float* x, const float* gamma,
                                  const float* beta, float* y, float* mean,
                                  float* rstd, float* mean_lo, int64_t N,
                                  int64_t C, int64_t HW, int64_t G, float eps,
                                  unsigned flags, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* Backward of soar_gn_silu_forward given upstream gradient dy, the forward
 * input x and the saved mean/rstd (and mean_lo).  SiLU is recomputed from
 * x (nothing but x and the statistics is saved by the forward).
 * mean_lo NULL: without SOAR_GN_SILU the backward recovers the residual
 * itself (its reduction pass also sums x - mean, whose unit mean is the
 * residual), so the results keep full accuracy when std << |mean|; with
 * SOAR_GN_SILU it is taken as 0 (pass mean_lo for such inputs).
 *   dgamma[c] += sum_{n,hw} dz * xhat,  dbeta[c] += sum_{n,hw} dz
 *   dx = rstd*(gamma_c*dz - (S1 + xhat*S2)/M) [+ dy] [+ previous dx]
 * with dz the gradient at the GroupNorm output, xhat = (x-mean)*rstd,
 * S1 = sum_{c in g} gamma_c*sum dz, S2 = sum_{c in g} gamma_c*sum dz*xhat.
 * dx, dgamma, dbeta may each be NULL (not wanted), as the reference guards
 * each parameter gradient on its own (normalization_kernels.cu:142-152,
 * 262-265).  dgamma/dbeta always accumulate (+=), summing over
 * samples, as the reference's parameter-gradient kernels do
 * (normalization_kernels.cu:151-152, tensor.cpp:173-192).
 * Replaces: silu_backward (cuda_kernels.hpp:20) followed by
 * group_norm_backward (:85-88), GroupNormNode::backward / SiLUNode::backward
 * (src/nn/layers.cpp:502-618, 749-771) and, with SOAR_GN_RESIDUAL, the
 * AddNode gradient merge (src/nn/blocks.cpp:28-31, tensor.cpp:194-213). */
SOAR_API int soar_gn_silu_backward(const float* dy, const float* x,
                                   const float* gamma, const float* beta,
                                   const float* mean, const float* rstd,
                                   const float* mean_lo, float* dx,
                                   float* dgamma, float* dbeta,
                                   int64_t N, int64_t C, int64_t HW,
                                   int64_t G, unsigned flags, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* ---- the reference's operator API, same argument meaning -------------- */
/* These take the reference's exact arguments (one sample, [C,H,W]); their
 * workspace is owned by the library (one buffer per device, grown on
 * demand with hipMalloc, kept until process exit), so concurrent calls on
 * different streams of one device must not overlap. */

/* Replaces: group_norm_forward (cuda_kernels.hpp:82-84,
 * normalization_kernels.cu:93-111).  gamma/beta nullable.  Saves the fp32
 * mean and rstd, as the reference does; the output uses the exact mean. */
SOAR_API int soar_group_norm_forward(const float* in, const float* gamma,
                                     const float* beta, float* out,
                                     float* saved_mean, float* saved_rstd,
                                     size_t num_groups, size_t C, size_t HW,
                                     float eps, void* stream);

/* Replaces: group_norm_backward (cuda_kernels.hpp:85-88,
 * normalization_kernels.cu:251-289).  grad_in, grad_gamma, grad_beta are
 * accumulated into (+=) and each may be NULL; gamma nullable.  The fp32
 * rounding residual of the saved mean is recovered from `in` (see
 * soar_gn_silu_backward), so dgamma and grad_in keep full accuracy when
 * std << |mean|, where the reference's fp32 path does not
 * (src/nn/layers.cpp:704-707). */
SOAR_API int soar_group_norm_backward(const float* grad_out, const float* in,
                                      const float* gamma,
                                      const float* saved_mean,
                                      const float* saved_rstd, float* grad_in,
                                      float* grad_gamma, float* grad_beta,
                                      size_t num_groups, size_t C, size_t HW,
                                      void* stream);

/* Bytes of the static device scratch behind
 * soar_group_norm_backward_noalloc, per device (held until process exit). */
#define SOAR_GN_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)

/* No counterpart in the reference: soar_group_norm_backward for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, results and accumulate
 * semantics as soar_group_norm_backward, and the same kernels, but the
 * workspace is a static device array of SOAR_GN_NOALLOC_SCRATCH_BYTES per
 * device instead of a library-owned hipMalloc buffer: the call allocates
 * nothing (no hipMalloc / hipFree, no stream or event creation).  A shape
 * whose workspace (soar_gn_workspace_bytes(1, C, HW, num_groups)) exceeds
 * the scratch is refused with SOAR_EINVAL.  Every call on one device shares
 * that device's scratch: calls that overlap in time on one device race. */
SOAR_API int soar_group_norm_backward_noalloc(const float* grad_out,
                                              const float* in,
                                              const float* gamma,
                                              const float* saved_mean,
                                              const float* saved_rstd,
                                              float* grad_in, float* grad_gamma,
                                              float* grad_beta,
                                              size_t num_groups, size_t C,
                                              size_t HW, void* stream);

/* Replaces: silu_forward (cuda_kernels.hpp:19): y = x/(1+exp(-x)). */
SOAR_API int soar_silu_forward(const float* x, float* y, size_t n,
                               void* stream);

/* Replaces: silu_backward (cuda_kernels.hpp:20):
 * grad_x += grad_y * s*(1 + x*(1-s)), s = sigmoid(x).  (The reference's
 * scalar kernel accumulates, its float4 kernel overwrites; every caller
 * passes a zeroed grad_x, where both agree.  This one accumulates.) */
SOAR_API int soar_silu_backward(const float* grad_y, const float* x,
                                float* grad_x, size_t n, void* stream);

/* Replaces: add_forward (cuda_kernels.hpp:15), tensor_add.comp: y = a + b. */
SOAR_API int soar_add_forward(const float* a, const float* b, float* y,
                              size_t n, void* stream);

/* Replaces: add_backward (cuda_kernels.hpp:16): grad_a += grad_y,
 * grad_b += grad_y; either may be NULL.  Also the device gradient
 * accumulate of Tensor::add_grad (tensor.cpp:183, 203). */
SOAR_API int soar_add_backward(const float* grad_y, float* grad_a,
                               float* grad_b, size_t n, void* stream);

/* Replaces: cuda_zero / cuda_fill (cuda_kernels.hpp:11-12). */
SOAR_API int soar_zero(float* ptr, size_t n, void* stream);
SOAR_API int soar_fill(float* ptr, float value, size_t n, void* stream);

/* ---- pointwise convolution, the producer of CBA's GroupNorm ---------- */
/* The 1x1 / stride 1 / no-padding / groups 1 convolution of CBA blocks
 * (Down.pw, LKR.pw1/pw2, Ctx.cv1/cv2; src/nn/blocks.cpp:429-480) is a GEMM
 * over the pixel axis; it runs on the fp32 matrix cores (v_mfma_f32_32x32x2
 * f32: fp32 products, fp32 accumulation).  weight is [C_out][C_in], bias
 * [C_out] or NULL; activations are [C][HW] per sample. */

/* out[co][p] = bias[co] + sum_ci weight[co][ci] * in[ci][p], one sample.
 * Replaces: conv2d_1x1_forward (cuda_kernels.hpp:57-58,
 * src/cuda/ops/convolution_kernels.cu:10-40), called by Conv2d::forward
 * (src/nn/layers.cpp:351-352) when groups == 1, k == 1, stride 1, pad 0. */
SOAR_API int soar_conv2d_1x1_forward(const float* in, const float* weight,
                                     const float* bias, float* out,
                                     size_t C_in, size_t C_out, size_t HW,
                                     void* stream);

/* z[n] = weight x[n] + bias for N samples at once (the batched form of
 * soar_conv2d_1x1_forward; no workspace).
 * Replaces: conv2d_1x1_forward (cuda_kernels.hpp:57-58) in a loop over the
 * samples of a batch. */
SOAR_API int soar_pw_conv_forward(const float* x, const float* weight,
                                  const float* bias, float* z, int64_t N,
                                  int64_t C_in, int64_t C_out, int64_t HW,
                                  void* stream);

/* Bytes of workspace soar_pw_conv_gn_silu_forward needs for this shape
 * (0 for an invalid or empty shape). */
SOAR_API size_t soar_pw_conv_gn_workspace_bytes(int64_t N, int64_t C_out,
                                                int64_t HW, int64_t G);

/* CBA forward of a pointwise convolution over N samples:
 *   z = conv1x1(x; weight, bias)            [N][C_out][HW]
 *   y = silu(GroupNorm_G(z; gamma, beta))   with SOAR_GN_SILU, else the
 *                                           GroupNorm alone (CBA, act=false)
 * The GroupNorm statistics of z are computed in the convolution's
 * epilogue, so z is written once and read once (by the apply) instead of
 * being read again for a statistics pass.  z, mean, rstd and mean_lo are
 * what soar_gn_silu_backward(dy, z, ...) needs for the backward of the
 * normalisation.  Flags: SOAR_GN_SILU only.
 * Replaces: CBA::forward (src/nn/blocks.cpp:442-445) = Conv2d::forward
 * (src/nn/layers.cpp:326-372) + GroupNorm::forward (layers.cpp:641-739)
 * + SiLU::forward (layers.cpp:778-800). */
SOAR_API int soar_pw_conv_gn_silu_forward(
    const float* x, const float* weight, const float* bias,
    const float* gamma, const float* beta, float* z, float* y, float* mean,
    float* rstd, float* mean_lo, int64_t N, int64_t C_in, int64_t C_out,
    int64_t HW, int64_t G, float eps, unsigned flags, void* workspace,
    size_t workspace_bytes, void* stream);

/* The same CBA forward followed by a residual add, y = (the output above)
 * + residual ([N][C_out][HW], e.g. the SOAR LKR block's input x:
 * blocks.cpp:469-475's x + pw2(pw1(dw(x)))), the add done by the apply pass
 * (one launch and two tensor passes fewer than the forward and an add).
 * Workspace as soar_pw_conv_gn_silu_forward.  No counterpart in the
 * reference (its LKR block adds after the CBA). */
SOAR_API int soar_pw_conv_gn_silu_add_forward(
    const float* x, const float* weight, const float* bias,
    const float* gamma, const float* beta, const float* residual, float* z,
    float* y, float* mean, float* rstd, float* mean_lo, int64_t N,
    int64_t C_in, int64_t C_out, int64_t HW, int64_t G, float eps,
    unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of workspace soar_pw_conv_backward needs (0 for a bad shape). */
SOAR_API size_t soar_pw_conv_backward_workspace_bytes(int64_t N, int64_t C_in,
                                                      int64_t C_out, int64_t HW);

/* Backward of the pointwise convolution over N samples, dz = dL/dz:
 *   dx   = W^T dz   [N][C_in][HW]; written, or added with
 *                   SOAR_GN_ACCUMULATE_DX; NULL skips it
 *   dw  += sum_n dz x^T  [C_out][C_in]; NULL skips it
 *   db  += sum_n,p dz    [C_out];       NULL skips it
 * dx runs on the same fp32 matrix-core kernel as the forward (with W^T);
 * dw is a split-K matrix-core product over pixel chunks whose fp32 partials
 * are added in a fixed order in float64, so results are reproducible.
 * Replaces: conv2d_1x1_backward (cuda_kernels.hpp:59-61,
 * src/cuda/ops/convolution_kernels.cu:42-133) as Conv2dNode::backward calls
 * it (src/nn/layers.cpp:34-85), batched over samples. */
SOAR_API int soar_pw_conv_backward(const float* dz, const float* x,
                                   const float* weight, float* dx,
                                   float* dweight, float* dbias, int64_t N,
                                   int64_t C_in, int64_t C_out, int64_t HW,
                                   unsigned flags, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* Reference signature, one sample: grad_in += W^T grad_out,
 * grad_weight += grad_out in^T, grad_bias += sum grad_out; any of the
 * three may be NULL.  Workspace owned by the library.
 * Replaces: conv2d_1x1_backward (cuda_kernels.hpp:59-61). */
SOAR_API int soar_conv2d_1x1_backward(const float* grad_out, const float* in,
                                      const float* weight, float* grad_in,
                                      float* grad_weight, float* grad_bias,
                                      size_t C_in, size_t C_out, size_t HW,
                                      void* stream);

/* Bytes of workspace soar_pw_cba_backward needs for this shape (0 for an
 * invalid or empty shape).  It assumes 16-byte aligned dy, z, x and dx. */
SOAR_API size_t soar_pw_cba_backward_workspace_bytes(int64_t N, int64_t C_in,
                                                     int64_t C_out, int64_t HW,
                                                     int64_t G);

/* Backward of a pointwise CBA block whose forward was
 * soar_pw_conv_gn_silu_forward(x, weight, NULL, gamma, beta, z, y, mean,
 * rstd, mean_lo, ...): with dz the GroupNorm(+SiLU) input gradient at z,
 *   dx      = W^T dz  [N][C_in][HW]; written, or added with
 *                     SOAR_GN_ACCUMULATE_DX; NULL skips it
 *   dweight += sum_n dz x^T  [C_out][C_in]; NULL skips it
 *   dgamma  += sum dz_gn * xhat, dbeta += sum dz_gn  [C_out]; each nullable
 * the same as soar_gn_silu_backward(dy, z, ..., dz, dgamma, dbeta) followed
 * by soar_pw_conv_backward(dz, x, weight, dx, dweight, NULL).  With
 * C_in and C_out multiples of 8 up to 64, HW % 4 == 0 and at least
 * SOAR_TUNE_PW_CBA_MIN samples
 * x pixels, one matrix-core kernel forms dz from z and dy in registers and
 * computes dx and the weight-gradient partials from it, so dz never
 * reaches HBM: z, dy and x are read once and dx written once after the
 * GroupNorm reduction pass.  Other shapes (or unaligned tensors with a
 * workspace large enough for it) run the two calls above with dz in the
 * workspace; a call for dgamma / dbeta alone runs the GroupNorm backward
 * only.  Flags: SOAR_GN_SILU, SOAR_GN_ACCUMULATE_DX.
 * Replaces: CBA backward as the autograd engine runs it, SiLUNode::backward
 * (src/nn/layers.cpp:749-771) + GroupNormNode::backward (:502-618) +
 * Conv2dNode::backward (:34-85) for CBA::forward (src/nn/blocks.cpp:442-445)
 * with a 1x1 convolution. */
SOAR_API int soar_pw_cba_backward(
    const float* dy, const float* z, const float* x, const float* weight,
    const float* gamma, const float* beta, const float* mean, const float* rstd,
    const float* mean_lo, float* dx, float* dweight, float* dgamma, float* dbeta,
    int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t G,
    unsigned flags, void* workspace, size_t workspace_bytes, void* stream);

/* ---- depthwise convolution (groups = C_in = C_out) ------------------- */
/* The K x K depthwise convolutions of CBA blocks: Down.dw (k3, stride 2),
 * LKR.dw (k5, k7), the Ctx branches (k3, dilation 1/3/5)
 * (src/nn/blocks.cpp:449-500).  x [N][C][H_in][W_in], y [N][C][H_out][W_out],
 * weight [C][K][K] (the reference's [C][1][K][K]), bias [C] or NULL.
 * y[n][c][yo][xo] = bias[c] + sum_(ky,kx) w[c][ky][kx] *
 *                   x[n][c][yo*stride - pad + ky*dil][xo*stride - pad + kx*dil],
 * taps outside the input skipped.  H_out/W_out are the caller's (Conv2d
 * computes (H + 2*pad - dil*(K-1) - 1)/stride + 1, layers.cpp:330-332).
 * Tiled LDS kernels for (K, stride, dil) = (3,1,1) (3,2,1) (5,1,1) (7,1,1)
 * (3,1,2) (3,1,3) (3,1,5); other shapes run generic kernels. */
SOAR_API int soar_dw_conv_forward(const float* x, const float* weight,
                                  const float* bias, float* y, int64_t N,
                                  int64_t C, int64_t H_in, int64_t W_in,
                                  int64_t H_out, int64_t W_out, int64_t K,
                                  int64_t pad, int64_t stride, int64_t dil,
                                  void* stream);

/* Bytes of workspace soar_dw_conv_gn_silu_forward needs for this shape (0
 * for an invalid or empty shape). */
SOAR_API size_t soar_dw_conv_gn_workspace_bytes(int64_t N, int64_t C,
                                                int64_t H_in, int64_t W_in,
                                                int64_t H_out, int64_t W_out,
                                                int64_t K, int64_t pad,
                                                int64_t stride, int64_t dil,
                                                int64_t G);

/* CBA forward of a depthwise convolution over N samples:
 *   z = bias + w (*) x   (as soar_dw_conv_forward, bit for bit)
 *   y = silu(GroupNorm_G(z)) (SOAR_GN_SILU) or GroupNorm_G(z), with mean,
 *       rstd, mean_lo (nullable) as soar_gn_silu_forward writes them.
 * For a shape with a tiled kernel, the convolution's epilogue computes the
 * GroupNorm statistics of its own outputs (each block's tile column as
 * float64 (mean, M2) partials in the workspace), so no separate statistics
 * pass re-reads z: the GroupNorm finish and apply follow directly.  Other
 * shapes, and units small enough for the one-launch GroupNorm, run the
 * convolution and then soar_gn_silu_forward.  mean / rstd match the
 * stand-alone forward's to float64 summation order.
 * Replaces: CBA::forward (src/nn/blocks.cpp:442-445) with a depthwise
 * Conv2d: Conv2d::forward (layers.cpp:353-355) + GroupNorm::forward
 * (:641-736) + SiLU::forward (:789-795). */
SOAR_API int soar_dw_conv_gn_silu_forward(
    const float* x, const float* weight, const float* bias, const float* gamma,
    const float* beta, float* z, float* y, float* mean, float* rstd,
    float* mean_lo, int64_t N, int64_t C, int64_t H_in, int64_t W_in,
    int64_t H_out, int64_t W_out, int64_t K, int64_t pad, int64_t stride,
    int64_t dil, int64_t G, float eps, unsigned flags, void* workspace,
    size_t workspace_bytes, void* stream);

/* Bytes of workspace soar_dw_conv_backward needs (0 is a valid answer: the
 * generic kernels need none; (size_t)-1 for an invalid shape). */
SOAR_API size_t soar_dw_conv_backward_workspace_bytes(
    int64_t N, int64_t C, int64_t H_in, int64_t W_in, int64_t H_out,
    int64_t W_out, int64_t K, int64_t stride, int64_t dil);

/* Backward over N samples: dx written (added with SOAR_GN_ACCUMULATE_DX),
 * dweight += and dbias += (summed over samples); any output may be NULL.
 * dweight/dbias come from per-tile partials added in a fixed order in
 * float64, so results are reproducible.
 * Replaces: conv2d_dw_backward (cuda_kernels.hpp:67-70,
 * src/cuda/ops/convolution_kernels.cu:184-333) as Conv2dNode::backward
 * calls it (src/nn/layers.cpp:73-77), batched over samples. */
SOAR_API int soar_dw_conv_backward(const float* dy, const float* x,
                                   const float* weight, float* dx,
                                   float* dweight, float* dbias, int64_t N,
                                   int64_t C, int64_t H_in, int64_t W_in,
                                   int64_t H_out, int64_t W_out, int64_t K,
                                   int64_t pad, int64_t stride, int64_t dil,
                                   unsigned flags, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* Bytes of workspace soar_dw_cba_backward needs for this shape (0 for an
 * invalid or empty shape). */
SOAR_API size_t soar_dw_cba_backward_workspace_bytes(
    int64_t N, int64_t C, int64_t H_in, int64_t W_in, int64_t H_out,
    int64_t W_out, int64_t K, int64_t pad, int64_t stride, int64_t dil,
    int64_t G);

/* Backward of a depthwise CBA block: z = dwconv(x; weight) without bias,
 * y = silu(GroupNorm_G(z)) (SOAR_GN_SILU) or GroupNorm_G(z); mean, rstd,
 * mean_lo are the GroupNorm forward's.  With dz the GroupNorm(+SiLU) input
 * gradient at z:
 *   dx      = the convolution's input gradient of dz; written, or added
 *             with SOAR_GN_ACCUMULATE_DX; NULL skips it
 *   dweight += its weight gradient [C][K][K]; NULL skips it
 *   dgamma  += sum dz_gn * xhat, dbeta += sum dz_gn  [C]; each nullable
 * the same as soar_gn_silu_backward(dy, z, ..., dz, dgamma, dbeta) followed
 * by soar_dw_conv_backward(dz, x, weight, dx, dweight, NULL, ...).  For a
 * stride-1 convolution with "same" padding, pad = (K-1)*dil/2, a
 * configuration with a tiled kernel (K = 3, 5, 7; K = 3 with dil 2, 3, 5)
 * and at least SOAR_TUNE_DW_CBA_MIN samples x pixels, one kernel forms dz
 * over each tile and its halo in LDS and computes dx and the
 * weight-gradient partials from it, so dz never reaches HBM.  Other calls
 * run the two calls above with dz in the workspace; a call for dgamma /
 * dbeta alone runs the GroupNorm backward only.
 * Flags: SOAR_GN_SILU, SOAR_GN_ACCUMULATE_DX.
 * Replaces: CBA backward as the autograd engine runs it, SiLUNode::backward
 * (src/nn/layers.cpp:749-771) + GroupNormNode::backward (:502-618) +
 * Conv2dNode::backward (:34-85) for CBA::forward (src/nn/blocks.cpp:442-445)
 * with a depthwise convolution. */
SOAR_API int soar_dw_cba_backward(
    const float* dy, const float* z, const float* x, const float* weight,
    const float* gamma, const float* beta, const float* mean, const float* rstd,
    const float* mean_lo, float* dx, float* dweight, float* dgamma, float* dbeta,
    int64_t N, int64_t C, int64_t H_in, int64_t W_in, int64_t H_out,
    int64_t W_out, int64_t K, int64_t pad, int64_t stride, int64_t dil,
    int64_t G, unsigned flags, void* workspace, size_t workspace_bytes,
    void* stream);

/* Runs every weight-gradient finish the calling thread's convolution
 * backward calls left pending (SOAR_DEFER_WEIGHT_FINISH) as one kernel
 * launch (several past 64 of them) on the stream they were queued on;
 * `stream` must be that stream (or the queue empty).  A call that queues a
 * finish on another stream, or one adding into weights already queued,
 * flushes the queue first.  No counterpart in the reference, whose layers
 * add their weight gradients in their own backward
 * (src/nn/layers.cpp:34-85, src/cuda/ops/convolution_kernels.cu:42-133);
 * it serves a training step that reads no weight gradient before its
 * clip (src/engine/trainer.cpp:110-220). */
SOAR_API int soar_weight_grad_flush(void* stream);

/* Weight-gradient finishes pending on the calling thread. */
SOAR_API size_t soar_weight_grad_pending(void);

/* Drops the calling thread's pending weight-gradient finishes without
 * running them: for a caller that abandons the backward pass that queued
 * them (an error part way through, a retry with a new workspace arena),
 * whose workspaces they read.  Their weight gradients keep whatever the
 * abandoned pass left.  A pending finish whose workspace is freed or
 * reused must be dropped before the next convolution backward call or
 * flush on the thread, which would otherwise run it. */
SOAR_API void soar_weight_grad_discard(void);

/* Reference signatures, one sample.
 * Replaces: conv2d_dw_forward (cuda_kernels.hpp:64-66,
 * convolution_kernels.cu:138-182), called by Conv2d::forward
 * (layers.cpp:353-355) when groups == C_in == C_out. */
SOAR_API int soar_conv2d_dw_forward(const float* in, const float* weight,
                                    const float* bias, float* out, size_t C,
                                    size_t H_in, size_t W_in, size_t H_out,
                                    size_t W_out, size_t K, size_t pad,
                                    size_t stride, size_t dil, void* stream);
/* grad_in +=, grad_weight +=, grad_bias += (any may be NULL); workspace
 * owned by the library.  Replaces: conv2d_dw_backward
 * (cuda_kernels.hpp:67-70). */
SOAR_API int soar_conv2d_dw_backward(const float* grad_out, const float* in,
                                     const float* weight, float* grad_in,
                                     float* grad_weight, float* grad_bias,
                                     size_t C, size_t H_in, size_t W_in,
                                     size_t H_out, size_t W_out, size_t K,
                                     size_t pad, size_t stride, size_t dil,
                                     void* stream);

/* ---- device arena (replaces VulkanBuffer / CudaMemoryPool storage) ---- */
/* One hipMalloc'd slab per arena, bump-allocated at `alignment` (a power
 * of two, 256 in the reference).  Allocations made before
 * soar_arena_freeze_static() are the static region (parameters and their
 * gradients); soar_arena_reset_dynamic() drops everything after it in O(1),
 * so the next step's allocations land at the same offsets.
 * Replaces: DeviceSlabSubAllocator (src/memory/device_slab.cpp:6-56,
 * include/soar/memory/device_slab.hpp:21-47) backed by device memory, in
 * place of VulkanBuffer (src/vulkan/buffer.cpp:8-75) and
 * CudaMemoryPool::allocate (src/cuda/cuda_allocator.cpp:24-77). */
typedef struct soar_arena soar_arena;

SOAR_API int soar_arena_create(size_t capacity_bytes, size_t alignment,
                               soar_arena** arena);
/* Zero bytes is an error (SOAR_EINVAL) as in device_slab.cpp:13-15;
 * exhaustion is SOAR_ENOMEM (device_slab.cpp:20-25). */
SOAR_API int soar_arena_alloc(soar_arena* arena, size_t bytes, void** dptr,
                              size_t* offset);
SOAR_API int soar_arena_freeze_static(soar_arena* arena);
SOAR_API int soar_arena_reset_dynamic(soar_arena* arena);
SOAR_API int soar_arena_info(const soar_arena* arena, size_t* capacity,
                             size_t* current_offset, size_t* static_boundary,
                             void** base);
SOAR_API int soar_arena_destroy(soar_arena* arena);

/* Host <-> device copies on `stream` (the Tensor::to_cuda / sync_to_host
 * boundary, src/tensor/tensor.cpp:146-165).  These synchronise `stream`
 * before returning, so the host buffer is free to reuse. */
SOAR_API int soar_memcpy_h2d(void* dst, const void* src, size_t bytes,
                             void* stream);
SOAR_API int soar_memcpy_d2h(void* dst, const void* src, size_t bytes,
                             void* stream);
/* Asynchronous copy on `stream` with no synchronisation: kind 0 host to
 * device, 1 device to host, 2 device to device.  The host buffer must stay
 * valid (and, for a copy recorded into a graph, pinned) until the stream
 * reaches the copy.  No counterpart in the reference. */
SOAR_API int soar_memcpy_async(void* dst, const void* src, size_t bytes,
                               int kind, void* stream);
/* Device-to-device copy, asynchronous on `stream` (Tensor::clone and the
 * per-sample slicing of Trainer::train_step, src/tensor/tensor.cpp and
 * src/engine/trainer.cpp:182, which call cudaMemcpyAsync DtoD). */
SOAR_API int soar_memcpy_d2d(void* dst, const void* src, size_t bytes,
                             void* stream);

/* ---- kernel timing (no counterpart in the reference) ------------------ */
/* When enabled, every kernel this library launches is bracketed by a pair
 * of hipEvents recorded on the launch stream.  soar_prof_summary()
 * synchronises those events and writes a JSON array
 * [{"kernel":name,"launches":n,"total_ms":t},...] into buf (truncated to
 * buflen), then clears the record.  Returns the number of kernels. */
SOAR_API int soar_prof_enable(int on);
SOAR_API int soar_prof_summary(char* buf, size_t buflen);

/* ---- tuning (no counterpart in the reference) ------------------------- */
/* Launch-shape knobs of the streaming kernels, set process-wide; the
 * defaults are the measured best on MI355X.  Values are validated. */
#define SOAR_TUNE_CHUNK 1    /* elements per block-chunk (multiple of 1024) */
#define SOAR_TUNE_REVERSE 2  /* 1: second passes walk chunks in reverse    */
#define SOAR_TUNE_NT_STORE 3 /* 1: non-temporal stores for y / dx          */
#define SOAR_TUNE_BATCH_MB 4 /* MiB per two-pass batch, 0 = whole tensor   */
#define SOAR_TUNE_STREAMS 5  /* 2: overlap batches on a helper stream      */
#define SOAR_TUNE_NT_LOAD 6  /* non-temporal loads: bit 0 in the second    */
                             /* passes, bit 1 in the first passes          */
#define SOAR_TUNE_CHUNK2 7   /* elements per block-chunk of apply / dx     */
#define SOAR_TUNE_PW_CHUNK 8 /* pixels per wave of the pointwise conv      */
                             /* (multiple of 128)                          */
#define SOAR_TUNE_SMALL_UNIT 9 /* units of <= this many elements run the   */
                               /* one-launch GroupNorm; 0 = never; the     */
                               /* default is 16384                         */
#define SOAR_TUNE_FOLD_MAX 11 /* units of <= this many partials (chunks,  */
                              /* or a depthwise forward's tile groups;    */
                              /* past 128 only units of <= 2^20 elements) */
                              /* fold the finish into the second pass     */
                              /* (one launch less per direction); 0 =     */
                              /* never, at most 4096, by default 2048     */
#define SOAR_TUNE_PW_SMALL 10 /* pointwise convs of <= this many multiply- */
                              /* adds (weight gradient: half as many) run */
                              /* the SIMT kernels; 0 = never; the default */
                              /* is 2^25                                  */
#define SOAR_TUNE_PW_SPLITK 12 /* most blocks the fused conv + GroupNorm  */
                               /* forward splits K over when its grid has  */
                               /* fewer than 256 tiles (fp32 slices in the */
                               /* workspace, added by a second kernel that */
                               /* also writes the statistics); 1 = never;  */
                               /* 1..8, the default is 8                   */
#define SOAR_TUNE_LOADS 13     /* 128-bit loads in flight per thread in */
                               /* the GroupNorm statistics and reduction */
                               /* passes: 4 or 8; results do not change  */
#define SOAR_TUNE_PW_WG_WAVES 14 /* pointwise weight gradient: waves per  */
                                 /* block that add their tiles in LDS     */
                                 /* before writing one partial: 1, 2, 4   */
                                 /* or 8; the default is 4                */
#define SOAR_TUNE_PW_WG_TARGET 15 /* waves the pointwise weight gradient  */
                                  /* sizes its pixel chunks for (at least */
                                  /* 64 pixels each): 256..2^20, default  */
                                  /* 2048; changes its workspace size     */
#define SOAR_TUNE_PW_CBA_MIN 16 /* pointwise CBA backward: the fused    */
                                /* kernel runs from this many samples x  */
                                /* pixels on (0 = never); default 2^14;  */
                                /* changes its workspace size            */
#define SOAR_TUNE_PW_CBA_BLOCKS 17 /* blocks the fused CBA backward sizes */
                                   /* its pixel chunks for: 64..2^20,    */
                                   /* default 256; changes its workspace  */
                                   /* size                                */
#define SOAR_TUNE_DW_CBA_MIN 18 /* depthwise CBA backward: the fused    */
                                /* kernel runs from this many samples x  */
                                /* pixels on (0 = never); changes its    */
                                /* workspace size                        */
#define SOAR_TUNE_NT_TAIL_MB 19 /* with SOAR_TUNE_NT_LOAD bit 1: MiB the  */
                                /* statistics / reduction passes read    */
                                /* last with cached loads (the second    */
                                /* pass walks in reverse and reads them  */
                                /* first, from the MALL)                 */
SOAR_API int soar_gn_tune(int key, int64_t value);
SOAR_API int64_t soar_gn_tune_get(int key);

#ifdef __cplusplus
}
#endif

#endif /* SOAR_GN_H */
