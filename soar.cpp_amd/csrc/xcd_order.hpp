// xcd_order.hpp - the XCD-aware block order of the convolution kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace soar {
namespace gn {

// Logical block of physical block b in a grid of nb blocks.  Workgroups are
// dealt to the 8 XCDs in turn (block b on XCD b % 8) and each XCD has its
// own L2.  Within each window of 256 blocks, XCD x takes 32 consecutive
// logical blocks (physical 256 w + 8 j + x -> logical 256 w + 32 x + j),
// while the blocks in flight still cover one compact band of the data.  A
// bijection on [0, nb); the last nb % 256 blocks keep their order.
//
// Depthwise tiles: adjacent tiles of a plane row share the 128-byte lines
// at their edges (the halo), so in the hardware order those lines came from
// the fabric twice (the k3 forward fetched 2.0x its input).  Measured at
// 64 x 2048^2, fwd / dgrad / wgrad: k3 0.463 / 0.469 / 0.480 ms in the
// hardware order, 0.429 / 0.447 / 0.439 ms here (1.11x / 1.08x / 1.03x
// fetched); a plain per-XCD split of the grid (XCD x one contiguous eighth)
// fetched as little but ran 0.476 / 0.494 / 0.417 ms, its XCDs far apart
// in the plane.  (Those figures are for 8 blocks per XCD in windows of 64.)
// Windows of 8 x 8 / 8 x 32 / 8 x 64 / 8 x 128 blocks on the final kernels
// (one box, two rounds, 64 x 2048^2): fused k3 CBA backward 0.849 / 0.823 /
// 0.824 / 0.848 ms, fused k7 1.116 / 1.099 / 1.097 / 1.096 ms, k3 weight
// gradient 0.442 / 0.377 / 0.380 / 0.392 ms, k3 forward 0.392 / 0.390 /
// 0.403 / 0.424 ms; the pointwise CBA step below 2.155 / 2.136 / 2.148 /
// 2.142 ms.  The halo lines at the edges of an XCD's run are fetched by two
// L2s, so longer runs fetch less, until the runs of the 8 XCDs lie too far
// apart in the plane.
//
// Pointwise pixel chunks share no lines, but a chunk reads and writes 512-
// byte runs of every channel plane, and the runs of consecutive chunks lie
// next to each other in the planes.  A probe that reads and writes 64
// planes 16 MiB apart in the streamed convolution's shape (one wave per
// SIMD, 1024-float chunks, 512-byte runs) took 490 us per GiB in the
// hardware order, 430 us in runs of 8 blocks per XCD and 424 us in runs of
// 32; the streamed forward with statistics at 64 -> 64 channels of 2048^2
// went from 486 to 468 and then 460 us, the fused CBA backward from 1.01 to
// 0.99 and then 0.97 ms.  The GroupNorm passes, whose blocks stream 32 KiB
// runs, gained nothing in runs of 8 (1.324 ms per config-3 step either
// way) and 1% in runs of 32 (1.326 -> 1.312 ms).
__device__ __forceinline__ int64_t xcd_block(int64_t b, int64_t nb) {
    constexpr int64_t kX = 8, kT = 32, kWin = kX * kT;  // XCDs, blocks per XCD run
    if (b >= nb / kWin * kWin) return b;
    const int64_t w = b / kWin, j = (b / kX) % kT, x = b % kX;
    return kWin * w + kT * x + j;
}

}  // namespace gn
}  // namespace soar
