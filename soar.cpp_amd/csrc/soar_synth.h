/*
 * soar_synth.h - seeded synthetic inputs on the device, for tests and the
 * benchmark (no counterpart in the reference, which draws its test inputs
 * from std::random_device).  Same generator as the CPU oracle: splitmix64
 * counter stream per (seed, tensor id), 53-bit uniforms, Box-Muller in
 * float64, rounded to fp32.  Tensor ids: x=1 gamma=2 beta=3 dy=4
 * outlier_mask=5 outlier_val=6.  Built into libsoar_synth.so, separate from
 * the product library.
 */
#ifndef SOAR_SYNTH_H
#define SOAR_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int soar_synth_normal(float* out, int64_t n, uint64_t seed, uint32_t stream_id,
                      double mean, double std_dev, void* stream);
int soar_synth_uniform(float* out, int64_t n, uint64_t seed, uint32_t stream_id,
                       double lo, double hi, void* stream);
int soar_synth_stress(float* out, int64_t n, uint64_t seed, double center,
                      double std_dev, double p, double out_mean, double out_std,
                      void* stream);
/* Plain 128-bit copy dst[i] = src[i] (n a multiple of 4, 16-byte aligned):
 * the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE. */
int soar_synth_copy(const float* src, float* dst, int64_t n, void* stream);
/* Streaming-ceiling kernels over n floats (a multiple of 4, 16-byte aligned
 * buffers of n floats each): kind 0 reads a, 1 copies a to out, 2 writes
 * out = a + b, 3 reads a and b.  One 256-thread block per 8192-float chunk,
 * like the library's streaming passes.  The read-only kinds leave out
 * unchanged (they write it only if a block's sum is exactly 1234.5). */
int soar_synth_stream(int kind, const float* a, const float* b, float* out,
                      int64_t n, void* stream);
/* The same four kinds in other launch shapes (test of whether the library's
 * shape or the memory system sets the ceilings): threads per block (64..1024,
 * a multiple of 64), loads = float4 loads in flight per thread and tensor
 * (2, 4 or 8), ntl / nts = non-temporal loads / stores.  persistent = 0:
 * one block per chunk of `size` floats (a multiple of 4, at least 4 *
 * threads); persistent = 1: a grid of `size` blocks striding over the
 * buffers in tiles of loads * threads float4s. */
int soar_synth_stream_shape(int kind, int persistent, int threads, int loads, int64_t size,
                            int ntl, int nts, const float* a, const float* b, float* out,
                            int64_t n, void* stream);
/* dst = src through the runtime's device-to-device hipMemcpyAsync. */
int soar_synth_memcpy_d2d(float* dst, const float* src, int64_t n, void* stream);
/* The pointwise convolution's access pattern over 64 planes of plane_floats
 * floats (a multiple of 1024), plane c at a + c * stride_floats (buffers of
 * 64 * stride_floats floats, 16-byte aligned): each block walks a 1024-float
 * window of every plane in 512-byte runs, all planes per run.  write = 1
 * copies a to out in that order, 0 only reads a. */
int soar_synth_planes(int write, const float* a, float* out, int64_t plane_floats,
                      int64_t stride_floats, void* stream);

#ifdef __cplusplus
}
#endif

#endif
