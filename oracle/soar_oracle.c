/*
 * soar_oracle.c - CPU oracle for the fused GroupNorm+SiLU path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and the
 * cpu_baseline leg of bench.py.  The product path never links or calls it.
 *
 * Build: see oracle/Makefile (gcc -O3 -std=c11, no -march, no fast-math,
 * matching the reference's Release flags, CMakeLists.txt:14).
 *
 * What pins each function (tests/test_oracle.py):
 *  - orc_gn_silu_fwd_f64 / orc_gn_silu_bwd_f64: torch float64 autograd
 *    fixtures (tests/golden/gn_silu_f64.npz), central finite differences,
 *    closed forms (constant group -> rstd = 1/sqrt(eps); two-valued group;
 *    sum_i dx_i = 0 per unit; sum_i xhat_i dx_i = rstd*S2*eps/(var+eps);
 *    dy = 0 -> zero grads; no-silu with dy = 1 -> dx = 0, dbeta = N*HW).
 *  - ref_*_f32: the reference test's own known-answer input
 *    (tests/test_operators.cpp:200-320, mt19937(999), U(-2,2), gamma=1.2,
 *    beta=-0.3, tol 1e-4 abs) against the float64 truth, and float64 truth
 *    at fp32-sized tolerances on seeded inputs.
 *  - orc_fill_*: splitmix64 published test vector (seed 1234567) and the
 *    moments of large samples.
 */
#define _POSIX_C_SOURCE 199309L
#include "soar_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ */
/* splitmix64 (Steele, Lea, Flood 2014; Vigna's reference constants)   */
/* ------------------------------------------------------------------ */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* Output number `ctr` (0-based) of a splitmix64 generator seeded with key:
 * the generator adds the golden gamma before every mix. */
uint64_t orc_splitmix64_at(uint64_t key, uint64_t ctr) {
    return mix64(key + (ctr + 1ULL) * 0x9E3779B97F4A7C15ULL);
}

uint64_t orc_stream_key(uint64_t seed, uint32_t stream) {
    return orc_splitmix64_at(seed, (uint64_t)stream);
}

static double uniform53(uint64_t bits) {
    return (double)(bits >> 11) * (1.0 / 9007199254740992.0);
}

/* Box-Muller pair p of stream `key`: (z0, z1) ~ iid N(0,1). */
static void box_muller(uint64_t key, int64_t p, double* z0, double* z1) {
    double u1 = 1.0 - uniform53(orc_splitmix64_at(key, 2ULL * (uint64_t)p));
    double u2 = uniform53(orc_splitmix64_at(key, 2ULL * (uint64_t)p + 1ULL));
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

void orc_fill_normal(float* out, int64_t n, uint64_t seed, uint32_t stream,
                     double mean, double std_dev) {
    uint64_t key = orc_stream_key(seed, stream);
    for (int64_t p = 0; 2 * p < n; ++p) {
        double z0, z1;
        box_muller(key, p, &z0, &z1);
        out[2 * p] = (float)(mean + std_dev * z0);
        if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std_dev * z1);
    }
}

void orc_fill_uniform(float* out, int64_t n, uint64_t seed, uint32_t stream,
                      double lo, double hi) {
    uint64_t key = orc_stream_key(seed, stream);
    for (int64_t i = 0; i < n; ++i)
        out[i] = (float)(lo + (hi - lo) * uniform53(orc_splitmix64_at(key, (uint64_t)i)));
}

void orc_fill_stress(float* out, int64_t n, uint64_t seed, double center,
                     double std_dev, double p, double out_mean, double out_std) {
    uint64_t kx = orc_stream_key(seed, 1), km = orc_stream_key(seed, 5),
             kv = orc_stream_key(seed, 6);
    for (int64_t q = 0; 2 * q < n; ++q) {
        double z[2], w[2];
        box_muller(kx, q, &z[0], &z[1]);
        box_muller(kv, q, &w[0], &w[1]);
        for (int k = 0; k < 2; ++k) {
            int64_t i = 2 * q + k;
            if (i >= n) break;
            double u = uniform53(orc_splitmix64_at(km, (uint64_t)i));
            out[i] = (u < p) ? (float)(out_mean + out_std * w[k])
                             : (float)(center + std_dev * z[k]);
        }
    }
}

/* ------------------------------------------------------------------ */
/* float64 truth                                                       */
/* ------------------------------------------------------------------ */

static int bad_shape(int64_t N, int64_t C, int64_t HW, int64_t G) {
    return N < 0 || C < 0 || HW < 0 || G <= 0 || (C % G) != 0;
}

/* Sum of a contiguous span in double, blocked so rounding grows with
 * log(n) rather than n. */
static double span_sum(const float* p, int64_t n) {
    double total = 0.0;
    for (int64_t b = 0; b < n; b += 4096) {
        int64_t e = b + 4096 < n ? b + 4096 : n;
        double s = 0.0;
        for (int64_t i = b; i < e; ++i) s += (double)p[i];
        total += s;
    }
    return total;
}

static double span_sqdev(const float* p, int64_t n, double m) {
    double total = 0.0;
    for (int64_t b = 0; b < n; b += 4096) {
        int64_t e = b + 4096 < n ? b + 4096 : n;
        double s = 0.0;
        for (int64_t i = b; i < e; ++i) {
            double d = (double)p[i] - m;
            s += d * d;
        }
        total += s;
    }
    return total;
}

int orc_gn_stats_f64(const float* x, int64_t N, int64_t C, int64_t HW,
                     int64_t G, double* mean, double* var) {
    if (bad_shape(N, C, HW, G)) return -1;
    int64_t M = (C / G) * HW;
    for (int64_t u = 0; u < N * G; ++u) {
        const float* p = x + u * M;
        double m = M ? span_sum(p, M) / (double)M : 0.0;
        double v = M ? span_sqdev(p, M, m) / (double)M : 0.0;
        if (mean) mean[u] = m;
        if (var) var[u] = v;
    }
    return 0;
}

static double sigmoid_f64(double z) { return 1.0 / (1.0 + exp(-z)); }

int orc_gn_silu_fwd_f64(const float* x, const float* gamma, const float* beta,
                        int64_t N, int64_t C, int64_t HW, int64_t G,
                        double eps, int apply_silu, int residual, double* y,
                        double* mean, double* rstd) {
    if (bad_shape(N, C, HW, G)) return -1;
    int64_t cpg = C / G;
    double* var = (double*)malloc(sizeof(double) * (size_t)(N * G + 1));
    double* mu = (double*)malloc(sizeof(double) * (size_t)(N * G + 1));
    if (!var || !mu) { free(var); free(mu); return -2; }
    orc_gn_stats_f64(x, N, C, HW, G, mu, var);
    for (int64_t u = 0; u < N * G; ++u) {
        double r = 1.0 / sqrt(var[u] + eps);
        if (mean) mean[u] = mu[u];
        if (rstd) rstd[u] = r;
        if (!y) continue;
        int64_t n = u / G, g = u % G;
        for (int64_t cg = 0; cg < cpg; ++cg) {
            int64_t c = g * cpg + cg;
            double gm = gamma ? (double)gamma[c] : 1.0;
            double bt = beta ? (double)beta[c] : 0.0;
            const float* xp = x + (n * C + c) * HW;
            double* yp = y + (n * C + c) * HW;
            for (int64_t i = 0; i < HW; ++i) {
                double z = gm * (((double)xp[i] - mu[u]) * r) + bt;
                double v = apply_silu ? z * sigmoid_f64(z) : z;
                yp[i] = residual ? v + (double)xp[i] : v;
            }
        }
    }
    free(var);
    free(mu);
    return 0;
}

int orc_gn_silu_bwd_f64(const float* dy, const float* x, const float* gamma,
                        const float* beta, const double* mean,
                        const double* rstd, int64_t N, int64_t C, int64_t HW,
                        int64_t G, int apply_silu, int residual, double* dx,
                        double* dgamma, double* dbeta) {
    if (bad_shape(N, C, HW, G)) return -1;
    int64_t cpg = C / G;
    double M = (double)(cpg * HW);
    /* per (n,c): a = sum dz, b = sum dz*xhat */
    double* a = (double*)calloc((size_t)(N * C + 1), sizeof(double));
    double* b = (double*)calloc((size_t)(N * C + 1), sizeof(double));
    if (!a || !b) { free(a); free(b); return -2; }
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t c = 0; c < C; ++c) {
            int64_t u = n * G + c / cpg;
            double gm = gamma ? (double)gamma[c] : 1.0;
            double bt = beta ? (double)beta[c] : 0.0;
            const float* xp = x + (n * C + c) * HW;
            const float* dp = dy + (n * C + c) * HW;
            double sa = 0.0, sb = 0.0;
            for (int64_t blk = 0; blk < HW; blk += 4096) {
                int64_t e = blk + 4096 < HW ? blk + 4096 : HW;
                double ta = 0.0, tb = 0.0;
                for (int64_t i = blk; i < e; ++i) {
                    double xh = ((double)xp[i] - mean[u]) * rstd[u];
                    double dz = (double)dp[i];
                    if (apply_silu) {
                        double z = gm * xh + bt, s = sigmoid_f64(z);
                        dz *= s * (1.0 + z * (1.0 - s));
                    }
                    ta += dz;
                    tb += dz * xh;
                }
                sa += ta;
                sb += tb;
            }
            a[n * C + c] = sa;
            b[n * C + c] = sb;
        }
    }
    if (dgamma || dbeta) {
        for (int64_t c = 0; c < C; ++c) {
            double sg = 0.0, sbt = 0.0;
            for (int64_t n = 0; n < N; ++n) {
                sbt += a[n * C + c];
                sg += b[n * C + c];
            }
            if (dgamma) dgamma[c] = sg;
            if (dbeta) dbeta[c] = sbt;
        }
    }
    if (dx) {
        for (int64_t u = 0; u < N * G; ++u) {
            int64_t n = u / G, g = u % G;
            double s1 = 0.0, s2 = 0.0;
            for (int64_t cg = 0; cg < cpg; ++cg) {
                int64_t c = g * cpg + cg;
                double gm = gamma ? (double)gamma[c] : 1.0;
                s1 += gm * a[n * C + c];
                s2 += gm * b[n * C + c];
            }
            for (int64_t cg = 0; cg < cpg; ++cg) {
                int64_t c = g * cpg + cg;
                double gm = gamma ? (double)gamma[c] : 1.0;
                double bt = beta ? (double)beta[c] : 0.0;
                const float* xp = x + (n * C + c) * HW;
                const float* dp = dy + (n * C + c) * HW;
                double* op = dx + (n * C + c) * HW;
                for (int64_t i = 0; i < HW; ++i) {
                    double xh = ((double)xp[i] - mean[u]) * rstd[u];
                    double dz = (double)dp[i];
                    if (apply_silu) {
                        double z = gm * xh + bt, s = sigmoid_f64(z);
                        dz *= s * (1.0 + z * (1.0 - s));
                    }
                    double v = rstd[u] * (gm * dz - (s1 + xh * s2) / M);
                    op[i] = residual ? v + (double)dp[i] : v;
                }
            }
        }
    }
    free(a);
    free(b);
    return 0;
}

/* ------------------------------------------------------------------ */
/* fp32 statement of the reference CPU path                            */
/* ------------------------------------------------------------------ */

/* GroupNorm::forward CPU branch, src/nn/layers.cpp:684-721: per group a
 * double sum / sum of squares, finished in float as
 * var = max(E[x^2] - mean^2, 0), rstd = 1/sqrt(var + eps); then
 * y = g*(x-mean)*rstd + b evaluated left to right. */
int ref_group_norm_forward_f32(const float* x, const float* gamma,
                               const float* beta, float* y, float* means,
                               float* rstds, int64_t C, int64_t HW,
                               int64_t G, float eps) {
    if (bad_shape(1, C, HW, G)) return -1;
    int64_t cpg = C / G;
    int64_t M = cpg * HW;
    for (int64_t grp = 0; grp < G; ++grp) {
        double sum = 0.0, sum_sq = 0.0;
        for (int64_t cg = 0; cg < cpg; ++cg) {
            int64_t c = grp * cpg + cg;
            for (int64_t sp = 0; sp < HW; ++sp) {
                float val = x[c * HW + sp];
                sum += val;
                sum_sq += (double)val * (double)val;
            }
        }
        float mean = (float)(sum / (double)M);
        float mean_sq = (float)(sum_sq / (double)M);
        float d = mean_sq - mean * mean;
        float var = d > 0.0f ? d : 0.0f;
        float rstd = 1.0f / sqrtf(var + eps);
        means[grp] = mean;
        rstds[grp] = rstd;
        for (int64_t cg = 0; cg < cpg; ++cg) {
            int64_t c = grp * cpg + cg;
            float g_val = gamma ? gamma[c] : 1.0f;
            float b_val = beta ? beta[c] : 0.0f;
            for (int64_t sp = 0; sp < HW; ++sp) {
                float val = x[c * HW + sp];
                y[c * HW + sp] = g_val * (val - mean) * rstd + b_val;
            }
        }
    }
    return 0;
}

/* SiLU::forward CPU branch, src/nn/layers.cpp:789-795. */
void ref_silu_forward_f32(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] / (1.0f + expf(-x[i]));
}

/* SiLUNode::backward CPU branch, src/nn/layers.cpp:760-769 (writes into a
 * freshly zeroed buffer, i.e. overwrites). */
void ref_silu_backward_f32(const float* grad_y, const float* x, float* grad_x,
                           int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float sig = 1.0f / (1.0f + expf(-x[i]));
        float dsilu = sig * (1.0f + x[i] * (1.0f - sig));
        grad_x[i] = grad_y[i] * dsilu;
    }
}

/* GroupNormNode::backward CPU branch, src/nn/layers.cpp:545-617: fp32
 * sequential sums; dgamma/dbeta per channel (:555-581), then per group
 * sum_dy / sum_dy_xhat and gx = (rstd/M)*(M*dy - sum_dy - xhat*sum_dy_xhat)
 * (:584-616).  grad_gamma/grad_beta/grad_x may each be NULL. */
int ref_group_norm_backward_f32(const float* go, const float* x,
                                const float* g, const float* means,
                                const float* rstds, float* gx, float* gw,
                                float* gb, int64_t C, int64_t HW, int64_t G) {
    if (bad_shape(1, C, HW, G)) return -1;
    int64_t cpg = C / G;
    int64_t M = cpg * HW;
    if (gw && gb) {
        for (int64_t grp = 0; grp < G; ++grp) {
            float mean = means[grp], rstd = rstds[grp];
            for (int64_t cg = 0; cg < cpg; ++cg) {
                int64_t c = grp * cpg + cg;
                float sum_w = 0.0f, sum_b = 0.0f;
                for (int64_t sp = 0; sp < HW; ++sp) {
                    float go_val = go[c * HW + sp];
                    float x_val = x[c * HW + sp];
                    sum_w += go_val * (x_val - mean) * rstd;
                    sum_b += go_val;
                }
                gw[c] = sum_w;
                gb[c] = sum_b;
            }
        }
    }
    if (gx) {
        for (int64_t grp = 0; grp < G; ++grp) {
            float mean = means[grp], rstd = rstds[grp];
            float sum_dy = 0.0f, sum_dy_xhat = 0.0f;
            for (int64_t cg = 0; cg < cpg; ++cg) {
                int64_t c = grp * cpg + cg;
                float g_val = g ? g[c] : 1.0f;
                for (int64_t sp = 0; sp < HW; ++sp) {
                    float dy = go[c * HW + sp] * g_val;
                    float xhat = (x[c * HW + sp] - mean) * rstd;
                    sum_dy += dy;
                    sum_dy_xhat += dy * xhat;
                }
            }
            for (int64_t cg = 0; cg < cpg; ++cg) {
                int64_t c = grp * cpg + cg;
                float g_val = g ? g[c] : 1.0f;
                for (int64_t sp = 0; sp < HW; ++sp) {
                    float dy = go[c * HW + sp] * g_val;
                    float xhat = (x[c * HW + sp] - mean) * rstd;
                    gx[c * HW + sp] = (rstd / (float)M) *
                                      ((float)M * dy - sum_dy - xhat * sum_dy_xhat);
                }
            }
        }
    }
    return 0;
}

/* add_tensors CPU branch, src/nn/blocks.cpp:57-64. */
void ref_add_f32(const float* a, const float* b, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = a[i] + b[i];
}

/* Tensor::add_grad / AutogradNode::add_grad_output CPU accumulate,
 * src/tensor/tensor.cpp:185-190, 205-211. */
void ref_accumulate_f32(const float* g, float* acc, int64_t n) {
    for (int64_t i = 0; i < n; ++i) acc[i] += g[i];
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* The reference's unfused GN -> SiLU [-> add] per sample, as CBA::forward
 * (src/nn/blocks.cpp:442-445) with the N>1 per-sample loop of
 * Trainer::train_step (src/engine/trainer.cpp:179-220).  Backward is
 * SiLUNode then GroupNormNode; parameter grads are summed over samples in
 * sample order as Tensor::add_grad does (clone, then +=); the residual
 * gradient dy is added once to the GN input gradient (AddNode,
 * src/nn/blocks.cpp:28-31). */
int ref_gn_silu_fwd_bwd_f32(const float* x, const float* gamma,
                            const float* beta, const float* dy, int64_t N,
                            int64_t C, int64_t HW, int64_t G, float eps,
                            int residual, float* gn_out, float* y,
                            float* means, float* rstds, float* dz, float* dx,
                            float* dgamma, float* dbeta, double* fwd_seconds,
                            double* bwd_seconds) {
    if (bad_shape(N, C, HW, G)) return -1;
    int64_t S = C * HW;
    double t0 = now_s();
    for (int64_t n = 0; n < N; ++n) {
        ref_group_norm_forward_f32(x + n * S, gamma, beta, gn_out + n * S,
                                   means + n * G, rstds + n * G, C, HW, G, eps);
        ref_silu_forward_f32(gn_out + n * S, y + n * S, S);
        if (residual) ref_add_f32(x + n * S, y + n * S, y + n * S, S);
    }
    double t1 = now_s();
    if (dy && dx) {
        float* gw = (float*)malloc(sizeof(float) * (size_t)(C + 1));
        float* gb = (float*)malloc(sizeof(float) * (size_t)(C + 1));
        if (!gw || !gb) { free(gw); free(gb); return -2; }
        for (int64_t n = 0; n < N; ++n) {
            ref_silu_backward_f32(dy + n * S, gn_out + n * S, dz + n * S, S);
            ref_group_norm_backward_f32(dz + n * S, x + n * S, gamma,
                                        means + n * G, rstds + n * G,
                                        dx + n * S, gw, gb, C, HW, G);
            if (residual) ref_accumulate_f32(dy + n * S, dx + n * S, S);
            if (n == 0) {
                if (dgamma) memcpy(dgamma, gw, sizeof(float) * (size_t)C);
                if (dbeta) memcpy(dbeta, gb, sizeof(float) * (size_t)C);
            } else {
                if (dgamma) ref_accumulate_f32(gw, dgamma, C);
                if (dbeta) ref_accumulate_f32(gb, dbeta, C);
            }
        }
        free(gw);
        free(gb);
    }
    double t2 = now_s();
    if (fwd_seconds) *fwd_seconds = t1 - t0;
    if (bwd_seconds) *bwd_seconds = t2 - t1;
    return 0;
}

/* ------------------------------------------------------------------ */
/* pointwise convolution                                               */
/* ------------------------------------------------------------------ */

int orc_conv1x1_fwd_f64(const float* x, const float* w, const float* b, int64_t N,
                        int64_t C_in, int64_t C_out, int64_t HW, double* y) {
    if (N < 0 || C_in <= 0 || C_out <= 0 || HW < 0) return -1;
    double* acc = (double*)malloc(sizeof(double) * (size_t)(HW > 0 ? HW : 1));
    if (!acc) return -2;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t co = 0; co < C_out; ++co) {
            const double bias = b ? (double)b[co] : 0.0;
            for (int64_t p = 0; p < HW; ++p) acc[p] = bias;
            for (int64_t ci = 0; ci < C_in; ++ci) {
                const double wv = (double)w[co * C_in + ci];
                const float* xr = x + (n * C_in + ci) * HW;
                for (int64_t p = 0; p < HW; ++p) acc[p] += wv * (double)xr[p];
            }
            memcpy(y + (n * C_out + co) * HW, acc, sizeof(double) * (size_t)HW);
        }
    }
    free(acc);
    return 0;
}

void ref_conv1x1_fwd_f32(const float* x, const float* w, const float* b, float* y,
                         int64_t C_in, int64_t C_out, int64_t HW) {
    for (int64_t idx = 0; idx < C_out * HW; ++idx) {
        const int64_t co = idx / HW, hw = idx % HW;
        float sum = b ? b[co] : 0.0f;
        const float* w_row = w + co * C_in;
        for (int64_t ci = 0; ci < C_in; ++ci) sum += w_row[ci] * x[ci * HW + hw];
        y[idx] = sum;
    }
}

int orc_conv1x1_bwd_f64(const float* dz, const float* x, const float* w, int64_t N,
                        int64_t C_in, int64_t C_out, int64_t HW, double* dx, double* dw,
                        double* db) {
    if (N < 0 || C_in <= 0 || C_out <= 0 || HW < 0) return -1;
    if (dx) {
        for (int64_t n = 0; n < N; ++n)
            for (int64_t ci = 0; ci < C_in; ++ci) {
                double* o = dx + (n * C_in + ci) * HW;
                for (int64_t p = 0; p < HW; ++p) o[p] = 0.0;
                for (int64_t co = 0; co < C_out; ++co) {
                    const double wv = (double)w[co * C_in + ci];
                    const float* g = dz + (n * C_out + co) * HW;
                    for (int64_t p = 0; p < HW; ++p) o[p] += wv * (double)g[p];
                }
            }
    }
    if (dw) {
        for (int64_t co = 0; co < C_out; ++co)
            for (int64_t ci = 0; ci < C_in; ++ci) {
                double acc = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const float* g = dz + (n * C_out + co) * HW;
                    const float* xr = x + (n * C_in + ci) * HW;
                    double part = 0.0;
                    for (int64_t p = 0; p < HW; ++p) part += (double)g[p] * (double)xr[p];
                    acc += part;
                }
                dw[co * C_in + ci] = acc;
            }
    }
    if (db) {
        for (int64_t co = 0; co < C_out; ++co) {
            double acc = 0.0;
            for (int64_t n = 0; n < N; ++n) acc += span_sum(dz + (n * C_out + co) * HW, HW);
            db[co] = acc;
        }
    }
    return 0;
}

void ref_conv1x1_bwd_f32(const float* grad_out, const float* in, const float* w,
                         float* grad_in, float* grad_weight, float* grad_bias,
                         int64_t C_in, int64_t C_out, int64_t HW) {
    if (grad_in && w) {
        for (int64_t idx = 0; idx < C_in * HW; ++idx) {
            const int64_t ci = idx / HW, hw = idx % HW;
            float sum = 0.0f;
            for (int64_t co = 0; co < C_out; ++co) sum += w[co * C_in + ci] * grad_out[co * HW + hw];
            grad_in[idx] += sum;
        }
    }
    if (grad_weight && in) {
        for (int64_t co = 0; co < C_out; ++co)
            for (int64_t ci = 0; ci < C_in; ++ci) {
                float sum = 0.0f;
                for (int64_t p = 0; p < HW; ++p) sum += grad_out[co * HW + p] * in[ci * HW + p];
                grad_weight[co * C_in + ci] += sum;
            }
    }
    if (grad_bias) {
        for (int64_t co = 0; co < C_out; ++co) {
            float sum = 0.0f;
            for (int64_t p = 0; p < HW; ++p) sum += grad_out[co * HW + p];
            grad_bias[co] += sum;
        }
    }
}

/* ------------------------------------------------------------------ */
/* depthwise convolution                                               */
/* ------------------------------------------------------------------ */

static int bad_dw(int64_t N, int64_t C, int64_t H_in, int64_t W_in, int64_t H_out,
                  int64_t W_out, int64_t K, int64_t pad, int64_t stride, int64_t dil) {
    return N < 0 || C < 0 || H_in < 0 || W_in < 0 || H_out < 0 || W_out < 0 || K <= 0 ||
           pad < 0 || stride <= 0 || dil <= 0;
}

int orc_dw_fwd_f64(const float* x, const float* w, const float* b, int64_t N, int64_t C,
                   int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                   int64_t pad, int64_t stride, int64_t dil, double* y) {
    if (bad_dw(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil)) return -1;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < C; ++c) {
            const float* xc = x + (n * C + c) * H_in * W_in;
            const float* wc = w + c * K * K;
            double* yc = y + (n * C + c) * H_out * W_out;
            for (int64_t yo = 0; yo < H_out; ++yo)
                for (int64_t xo = 0; xo < W_out; ++xo) {
                    double acc = b ? (double)b[c] : 0.0;
                    for (int64_t ky = 0; ky < K; ++ky) {
                        const int64_t yi = yo * stride - pad + ky * dil;
                        if (yi < 0 || yi >= H_in) continue;
                        for (int64_t kx = 0; kx < K; ++kx) {
                            const int64_t xi = xo * stride - pad + kx * dil;
                            if (xi < 0 || xi >= W_in) continue;
                            acc += (double)wc[ky * K + kx] * (double)xc[yi * W_in + xi];
                        }
                    }
                    yc[yo * W_out + xo] = acc;
                }
        }
    return 0;
}

int orc_dw_bwd_f64(const float* dy, const float* x, const float* w, int64_t N, int64_t C,
                   int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                   int64_t pad, int64_t stride, int64_t dil, double* dx, double* dw, double* db) {
    if (bad_dw(N, C, H_in, W_in, H_out, W_out, K, pad, stride, dil)) return -1;
    if (dx)
        for (int64_t i = 0; i < N * C * H_in * W_in; ++i) dx[i] = 0.0;
    if (dw)
        for (int64_t i = 0; i < C * K * K; ++i) dw[i] = 0.0;
    if (db)
        for (int64_t i = 0; i < C; ++i) db[i] = 0.0;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t c = 0; c < C; ++c) {
            const float* xc = x + (n * C + c) * H_in * W_in;
            const float* gc = dy + (n * C + c) * H_out * W_out;
            const float* wc = w + c * K * K;
            for (int64_t yo = 0; yo < H_out; ++yo)
                for (int64_t xo = 0; xo < W_out; ++xo) {
                    const double g = (double)gc[yo * W_out + xo];
                    if (db) db[c] += g;
                    for (int64_t ky = 0; ky < K; ++ky) {
                        const int64_t yi = yo * stride - pad + ky * dil;
                        if (yi < 0 || yi >= H_in) continue;
                        for (int64_t kx = 0; kx < K; ++kx) {
                            const int64_t xi = xo * stride - pad + kx * dil;
                            if (xi < 0 || xi >= W_in) continue;
                            if (dx)
                                dx[(n * C + c) * H_in * W_in + yi * W_in + xi] +=
                                    g * (double)wc[ky * K + kx];
                            if (dw) dw[c * K * K + ky * K + kx] += g * (double)xc[yi * W_in + xi];
                        }
                    }
                }
        }
    return 0;
}

void ref_dw_fwd_f32(const float* x, const float* w, const float* b, float* y, int64_t C,
                    int64_t H_in, int64_t W_in, int64_t H_out, int64_t W_out, int64_t K,
                    int64_t pad, int64_t stride, int64_t dil) {
    for (int64_t idx = 0; idx < C * H_out * W_out; ++idx) {
        const int64_t w_out = idx % W_out, t = idx / W_out;
        const int64_t h_out = t % H_out, c = t / H_out;
        float sum = b ? b[c] : 0.0f;
        const float* wc = w + c * K * K;
        const float* in_c = x + c * H_in * W_in;
        const int64_t hb = h_out * stride - pad, wb = w_out * stride - pad;
        for (int64_t kh = 0; kh < K; ++kh) {
            const int64_t hi = hb + kh * dil;
            if (hi < 0 || hi >= H_in) continue;
            for (int64_t kw = 0; kw < K; ++kw) {
                const int64_t wi = wb + kw * dil;
                if (wi >= 0 && wi < W_in) sum += in_c[hi * W_in + wi] * wc[kh * K + kw];
            }
        }
        y[idx] = sum;
    }
}

void ref_dw_bwd_f32(const float* dy, const float* x, const float* w, float* grad_in,
                    float* grad_weight, float* grad_bias, int64_t C, int64_t H_in, int64_t W_in,
                    int64_t H_out, int64_t W_out, int64_t K, int64_t pad, int64_t stride,
                    int64_t dil) {
    if (grad_in && w) {
        for (int64_t idx = 0; idx < C * H_in * W_in; ++idx) {
            const int64_t wi = idx % W_in, t = idx / W_in;
            const int64_t hi = t % H_in, c = t / H_in;
            float sum = 0.0f;
            const float* wc = w + c * K * K;
            const float* go = dy + c * H_out * W_out;
            for (int64_t kh = 0; kh < K; ++kh) {
                const int64_t nh = hi + pad - kh * dil;
                if (nh < 0 || nh % stride) continue;
                const int64_t ho = nh / stride;
                if (ho >= H_out) continue;
                for (int64_t kw = 0; kw < K; ++kw) {
                    const int64_t nw = wi + pad - kw * dil;
                    if (nw < 0 || nw % stride) continue;
                    const int64_t wo = nw / stride;
                    if (wo < W_out) sum += go[ho * W_out + wo] * wc[kh * K + kw];
                }
            }
            grad_in[idx] += sum;
        }
    }
    if (grad_weight && x) {
        for (int64_t p = 0; p < C * K * K; ++p) {
            const int64_t kw = p % K, t = p / K, kh = t % K, c = t / K;
            const float* go = dy + c * H_out * W_out;
            const float* xc = x + c * H_in * W_in;
            float sum = 0.0f;
            for (int64_t i = 0; i < H_out * W_out; ++i) {
                const int64_t ho = i / W_out, wo = i % W_out;
                const int64_t hi = ho * stride - pad + kh * dil, wi = wo * stride - pad + kw * dil;
                if (hi >= 0 && hi < H_in && wi >= 0 && wi < W_in) sum += go[i] * xc[hi * W_in + wi];
            }
            grad_weight[p] += sum;
        }
    }
    if (grad_bias) {
        for (int64_t c = 0; c < C; ++c) {
            float sum = 0.0f;
            for (int64_t i = 0; i < H_out * W_out; ++i) sum += dy[c * H_out * W_out + i];
            grad_bias[c] += sum;
        }
    }
}
