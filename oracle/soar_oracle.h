/*
 * soar_oracle.h - CPU oracle for the fused GroupNorm+SiLU path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this library: it is the checker that tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg compare the HIP kernels against.
 *
 * Two families of functions live here:
 *
 *  orc_*_f64  float64 "truth": two-pass statistics and the exact derivative
 *             of y = silu(gamma*(x-mean)*rstd + beta) [+ x].  Parity gates
 *             compare the GPU path against these.
 *
 *  ref_*_f32  a statement, in fp32 with the same operation order, of the
 *             reference's CPU loops (pomagrenate/soar.cpp src/nn/layers.cpp,
 *             src/nn/blocks.cpp).  This is the "port" CPU baseline and the
 *             second column of every parity report.
 *
 * Layout: fp32 NCHW contiguous; a "unit" is one (n, g) reduction domain of
 * M = (C/G)*HW contiguous elements; mean/rstd are indexed [n*G + g].
 *
 * Every function's header comment cites the reference lines it follows and
 * the test that pins it.
 */
#ifndef SOAR_ORACLE_H
#define SOAR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic inputs (splitmix64 -> 53-bit uniform -> Box-Muller) ---- */

/* splitmix64 output function applied to counter `ctr` of stream `key`. */
uint64_t orc_splitmix64_at(uint64_t key, uint64_t ctr);
/* Key for (seed, tensor stream id); stream ids: x=1 gamma=2 beta=3 dy=4
 * outlier_mask=5 outlier_val=6. */
uint64_t orc_stream_key(uint64_t seed, uint32_t stream);
/* out[i] = mean + std * N(0,1), pairs (2p, 2p+1) from one Box-Muller draw. */
void orc_fill_normal(float* out, int64_t n, uint64_t seed, uint32_t stream,
                     double mean, double std_dev);
/* out[i] = lo + (hi - lo) * U[0,1). */
void orc_fill_uniform(float* out, int64_t n, uint64_t seed, uint32_t stream,
                      double lo, double hi);
/* Stress input: x = center + N(0, std); with probability p per element the
 * value is replaced by out_mean + N(0, out_std). */
void orc_fill_stress(float* out, int64_t n, uint64_t seed, double center,
                     double std_dev, double p, double out_mean, double out_std);

/* ---- float64 truth ---- */

/* Two-pass mean and biased variance of every (n,g) unit. */
int orc_gn_stats_f64(const float* x, int64_t N, int64_t C, int64_t HW,
                     int64_t G, double* mean, double* var);

/* y = silu(gamma_c*(x-mean)*rstd + beta_c) (or without silu) [+ x].
 * gamma/beta may be NULL (1 / 0).  y may be NULL (stats only). */
int orc_gn_silu_fwd_f64(const float* x, const float* gamma, const float* beta,
                        int64_t N, int64_t C, int64_t HW, int64_t G,
                        double eps, int apply_silu, int residual, double* y,
                        double* mean, double* rstd);

/* Exact backward of orc_gn_silu_fwd_f64 at (mean, rstd) from the same call.
 * dx may be NULL; dgamma/dbeta are written (not accumulated), may be NULL. */
int orc_gn_silu_bwd_f64(const float* dy, const float* x, const float* gamma,
                        const float* beta, const double* mean,
                        const double* rstd, int64_t N, int64_t C, int64_t HW,
                        int64_t G, int apply_silu, int residual, double* dx,
                        double* dgamma, double* dbeta);

/* ---- fp32 statement of the reference CPU path (one sample, [C,H,W]) ---- */

int ref_group_norm_forward_f32(const float* x, const float* gamma,
                               const float* beta, float* y, float* means,
                               float* rstds, int64_t C, int64_t HW,
                               int64_t G, float eps);
void ref_silu_forward_f32(const float* x, float* y, int64_t n);
void ref_silu_backward_f32(const float* grad_y, const float* x, float* grad_x,
                           int64_t n);
int ref_group_norm_backward_f32(const float* grad_out, const float* x,
                                const float* gamma, const float* means,
                                const float* rstds, float* grad_x,
                                float* grad_gamma, float* grad_beta,
                                int64_t C, int64_t HW, int64_t G);
void ref_add_f32(const float* a, const float* b, float* y, int64_t n);
void ref_accumulate_f32(const float* g, float* acc, int64_t n);

/* The reference's unfused GN -> SiLU [-> residual add] sequence over N
 * samples (per-sample loop, dgamma/dbeta summed over samples).  `gn_out`,
 * `silu_out`, `dz` are caller scratch of N*C*HW floats (dz may alias
 * nothing else).  dgamma/dbeta are written. */
int ref_gn_silu_fwd_bwd_f32(const float* x, const float* gamma,
                            const float* beta, const float* dy, int64_t N,
                            int64_t C, int64_t HW, int64_t G, float eps,
                            int residual, float* gn_out, float* y,
                            float* means, float* rstds, float* dz, float* dx,
                            float* dgamma, float* dbeta, double* fwd_seconds,
                            double* bwd_seconds);

/* ---- pointwise (1x1) convolution, the producer of CBA's GroupNorm ---- */

/* float64 truth: y[n][co][p] = sum_ci w[co][ci] * x[n][ci][p] + b[co]
 * (b may be NULL).  y is double[N*C_out*HW]. */
int orc_conv1x1_fwd_f64(const float* x, const float* w, const float* b, int64_t N,
                        int64_t C_in, int64_t C_out, int64_t HW, double* y);
/* fp32 statement of the reference's k_conv2d_1x1_forward
 * (src/cuda/ops/convolution_kernels.cu:10-31): sum = bias, then
 * sum += w*x over ci in order, one sample. */
void ref_conv1x1_fwd_f32(const float* x, const float* w, const float* b,
                         float* y, int64_t C_in, int64_t C_out, int64_t HW);

/* float64 truth of the backward, N samples: dx = W^T dz, dw = sum_n dz x^T,
 * db = sum_n,p dz.  Outputs are written (not accumulated); any may be NULL. */
int orc_conv1x1_bwd_f64(const float* dz, const float* x, const float* w, int64_t N,
                        int64_t C_in, int64_t C_out, int64_t HW, double* dx, double* dw,
                        double* db);
/* fp32 statement of the reference's conv2d_1x1_backward kernels
 * (src/cuda/ops/convolution_kernels.cu:42-133), one sample, accumulating:
 * grad_in[ci][p] += sum_co w[co][ci]*go[co][p] (co ascending),
 * grad_weight[co][ci] += sum_p go[co][p]*x[ci][p], grad_bias[co] += sum_p go.
 * Pointers may be NULL (that gradient is skipped). */
void ref_conv1x1_bwd_f32(const float* grad_out, const float* in, const float* w,
                         float* grad_in, float* grad_weight, float* grad_bias,
                         int64_t C_in, int64_t C_out, int64_t HW);

/* ---- depthwise convolution (groups = C_in = C_out) ---- */

/* float64 truth, N samples: y[n][c][yo][xo] = b[c] + sum_(ky,kx)
 * w[c][ky][kx] * x[n][c][yo*s - pad + ky*d][xo*s - pad + kx*d], taps outside
 * the input skipped (zero padding).  b may be NULL. */
int orc_dw_fwd_f64(const float* x, const float* w, const float* b, int64_t N, int64_t C,
                   int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                   int64_t pad, int64_t stride, int64_t dil, double* y);
/* float64 truth of the backward: dx (scatter of dy through the taps),
 * dw[c][ky][kx] = sum_(n,yo,xo) dy * x at the tap, db[c] = sum dy; written,
 * any may be NULL. */
int orc_dw_bwd_f64(const float* dy, const float* x, const float* w, int64_t N, int64_t C,
                   int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                   int64_t pad, int64_t stride, int64_t dil, double* dx, double* dw, double* db);
/* fp32 statements of the reference's depthwise kernels, one sample
 * (src/cuda/ops/convolution_kernels.cu:138-333): forward (sum = bias, taps
 * in ky, kx order), and the accumulating backward (grad_in += gather over
 * taps; grad_weight += per-tap sums; grad_bias += sum).  NULL skips. */
void ref_dw_fwd_f32(const float* x, const float* w, const float* b, float* y, int64_t C,
                    int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                    int64_t pad, int64_t stride, int64_t dil);
void ref_dw_bwd_f32(const float* dy, const float* x, const float* w, float* grad_in,
                    float* grad_weight, float* grad_bias, int64_t C, int64_t H_in, int64_t W_in,
                    int64_t H_out, int64_t W_out, int64_t K, int64_t pad, int64_t stride,
                    int64_t dil);

#ifdef __cplusplus
}
#endif

#endif /* SOAR_ORACLE_H */
