// gn_internal.hpp - launch plans and launchers shared by the HIP kernels
// (gn_kernels.hip, elementwise.hip) and the C-ABI (capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace soar {
namespace gn {

// Launch geometry of the streaming kernels.  Every (n, c) plane of HW
// floats is cut into `cpp` chunks of `chunk` floats (the last one ragged);
// one 256-thread block streams one chunk.  Blocks are numbered
// plane * cpp + chunk_in_plane, so unit u = (n, g) owns the contiguous
// block range [u*cpg*cpp, (u+1)*cpg*cpp).
//
// Units are processed in batches: both passes of a batch (statistics then
// apply; reduction then dx) run before the next batch starts, so the second
// pass re-reads data the first pass just brought into the 256 MB MALL
// instead of streaming the whole tensor from HBM twice.
struct Plan {
    int64_t N = 0, C = 0, HW = 0, G = 0, cpg = 0;
    int64_t planes = 0;      // N * C
    int64_t units = 0;       // N * G
    int64_t chunk = 0;       // floats per block-chunk (first passes)
    int64_t cpp = 0;         // chunks per plane
    int64_t blocks = 0;      // planes * cpp
    int64_t chunk2 = 0;      // floats per block-chunk of the second passes
    int64_t cpp2 = 0;        // (apply / dx), which need no partials and
    int64_t blocks2 = 0;     // so may cut the planes differently
    int64_t upb_fwd = 0;     // units per forward batch
    int64_t upb_bwd = 0;     // units per backward batch
    bool vec4 = false;       // float4 path (HW % 4 == 0 and 16-byte pointers)
    int loads = 4;           // 128-bit loads in flight per thread, first passes
    bool ntl1 = false;       // non-temporal loads in the first passes ...
    int64_t nt_tail = 0;     // ... except for their last this many bytes read
};

// Defaults measured on MI355X at 1x64x2048^2, fwd+bwd per step:
//   chunk 8192, forward order, cached stores            1.541 ms
//   + reverse order + non-temporal stores                1.469 ms
//   + non-temporal loads in the second passes            1.447 ms
//   chunk 16384 / 32768                                  +1.5% / +3%
//   unit batches of 64 / 128 / 256 MiB (with nt loads)   1.525 / 1.475 /
//                                                        1.465 ms
//   same batches pipelined on two streams                1.740 / 1.628 /
//                                                        1.544 ms
// (each extra pair of launches costs ~2.7 us, more than the MALL saves).
// Later, with the first passes' load policy (one box, two runs each):
//   cached loads in the first passes                     1.429 ms
//   non-temporal loads there                             1.395 ms
//   non-temporal except the last 64 / 128 / 192 / 256 /
//   384 MiB read, which the reverse-walking second pass
//   then reads from the MALL                             1.393 / 1.384 /
//                                                        1.378 / 1.369 /
//                                                        1.390 ms
struct Tuning {
    int64_t chunk = 8192;     // floats per block-chunk, multiple of 1024
    int64_t chunk2 = 4096;    // same for the second passes (128-thread
                              // blocks; 2.5-3.5% faster there than 256 / 8192)
    int reverse = 1;          // second passes walk a batch's blocks in
                              // reverse, starting on what was read last
    int nt_store = 1;         // non-temporal stores of y / dx
    int64_t batch_mb = 0;     // MiB read by the first pass of a batch
                              // (0: the whole tensor is one batch)
    int streams = 1;          // 2: pipeline batches over a helper stream
    int nt_load = 3;          // non-temporal loads: bit 0 in the second passes
                              // (apply / dx), bit 1 in the first passes
                              // (statistics / reduction) except their tail:
    int64_t nt_tail_mb = 256; // MiB the first passes read last with cached
                              // loads (the reverse-walking second pass reads
                              // them first, from the MALL)
    int64_t pw_chunk = 1024;  // pixels per wave of the pointwise convolution
                              // (multiple of 128); also its GroupNorm
                              // partials' chunk
    int64_t small_unit = 16384;  // units of at most this many elements run
                                 // the one-launch GroupNorm (0: never); one
                                 // block per unit, so larger units stream
                                 // faster over many blocks (Nano 512^2 train
                                 // step: 3.73 ms at 32768, 3.64 at 16384)
    int64_t fold_max = 2048;     // units of at most this many partials (one
                                 // batch; past 128 only units of at most
                                 // 2^20 elements) fold the finish into the
                                 // second pass (0: never; at most 4096)
    int64_t pw_small = 1 << 25;  // pointwise convolutions of at most this
                                 // many multiply-adds (weight gradient: half
                                 // as many) run the SIMT kernels (0: never)
    int64_t pw_kz = 8;           // most blocks a small-grid pointwise
                                 // convolution splits K over (1: never)
    int loads = 4;               // 128-bit loads in flight per thread in the
                                 // first passes (statistics, reduction): 4 or 8
    int pw_wg_waves = 4;         // pointwise weight gradient: waves per block
                                 // that add their tiles before writing one
                                 // partial (1, 2, 4 or 8)
    int64_t pw_wg_target = 2048;  // and the waves its pixel chunks aim for
    int64_t pw_cba_min = 16384;  // pointwise CBA backward: samples x pixels
                                 // from which the fused kernel runs (0:
                                 // never); Nano train step with graphs at
                                 // 2^14 / 2^16 / 2^17 / never: 512^2 2.73 /
                                 // 2.92 / 2.90 / 2.96 ms, 1024^2 4.34 /
                                 // 4.36 / 4.45 / 4.54 ms
    int64_t dw_cba_min = 16384;  // depthwise CBA backward: samples x pixels
                                 // from which the fused kernel runs (0:
                                 // never)
    int64_t pw_cba_blocks = 256;  // and the blocks its pixel chunks aim for
                                  // (one per CU: at 64 -> 64 channels over
                                  // 2048^2 pixels 1.03 ms, 1.13 at 512,
                                  // 1.19 at 1024)
};

constexpr int kThreads = 256;   // first passes (stats, reduction)
// Second passes: threads per block and 128-bit loads per tensor a thread
// keeps in flight, for the apply (k_apply) and the dx pass (k_bwd_dx).  At
// the default 4096-float chunks both load a thread's whole share of its
// chunk in one batch (1 GiB tensors: apply 128 x 8 337 us, 512 x 2 336 us
// but slower at 256 MiB tensors; dx 128 x 8 520 us, 512 x 2 505 us).
#ifndef SOAR_GN_THREADS2
#define SOAR_GN_THREADS2 128
#endif
#ifndef SOAR_GN_LOADS2
#define SOAR_GN_LOADS2 8
#endif
#ifndef SOAR_GN_THREADS_DX
#define SOAR_GN_THREADS_DX 512
#endif
#ifndef SOAR_GN_LOADS_DX
#define SOAR_GN_LOADS_DX 2
#endif
constexpr int kThreads2 = SOAR_GN_THREADS2;  // apply
constexpr int kLoads2 = SOAR_GN_LOADS2;
constexpr int kThreadsDx = SOAR_GN_THREADS_DX;  // dx
constexpr int kLoadsDx = SOAR_GN_LOADS_DX;

// Plan for a non-empty tensor.  Returns false if the grid would not fit.
bool make_plan(int64_t N, int64_t C, int64_t HW, int64_t G,
               const Tuning& t, Plan* p);
size_t workspace_bytes(const Plan& p);

struct FwdArgs {
    const float* x;
    const float* gamma;  // nullable
    const float* beta;   // nullable
    float* y;
    float* mean;
    float* rstd;
    float* mean_lo;  // nullable: mean - (float)mean
    float eps;
    unsigned flags;
    void* ws;
    // with SOAR_GN_RESIDUAL: the tensor added to the output (x itself when
    // null); the one-launch small-unit kernels take x only
    const float* res = nullptr;
};

struct BwdArgs {
    const float* dy;
    const float* x;
    const float* gamma;  // nullable
    const float* beta;   // nullable
    const float* mean;
    const float* rstd;
    const float* mean_lo;  // nullable (treated as 0)
    float* dx;      // nullable
    float* dgamma;  // nullable (with dbeta)
    float* dbeta;
    unsigned flags;
    void* ws;
};

hipError_t launch_forward(const Plan& p, const Tuning& t, const FwdArgs& a,
                          hipStream_t s);
hipError_t launch_backward(const Plan& p, const Tuning& t, const BwdArgs& a,
                           hipStream_t s);

// True when the backward of this plan runs the one-launch small-unit kernel.
bool backward_is_small(const Plan& p, const Tuning& t);
// The backward's reduction and its finish over every unit (one batch), no
// dx pass: leaves per-plane (sum dz, sum dz xhat) and per-unit (S1, S2) in
// the workspace for a fused consumer.  mean_lo is the residual the dx
// arithmetic must use (the workspace's recovered one when the caller saved
// none and there is no SiLU).
// With `fold`, only the reduction runs: plane_sums and unit_sums are null
// and the consumer forms both from the chunk partials `part` (cpp per
// plane) with bwd_plane_sums / bwd_unit_sums, the finish's own arithmetic.
struct BwdSums {
    const double2* plane_sums;  // [N * C]
    const double2* unit_sums;   // [N * G]
    const float* mean_lo;       // [N * G], nullable
    const double2* part;        // [N * C][cpp] (fold)
    int64_t cpp;
};
hipError_t launch_backward_sums(const Plan& p, const BwdArgs& a, hipStream_t s, BwdSums* out,
                                bool fold = false);
// True if a consumer whose blocks each fold `planes` planes' partials
// (at most kFoldPlanes) may take the sums unfinished: the mean residual is
// not recovered and the partials fit the folded-finish limits.
constexpr int64_t kFoldPlanes = 64;
bool backward_sums_foldable(const Plan& p, const Tuning& t, const BwdArgs& a, int64_t planes);

// GroupNorm forward whose chunk partials are already in the workspace (the
// pointwise convolution wrote them): the finish, then the apply, over all
// units.
hipError_t launch_forward_from_partials(const Plan& p, const Tuning& t, const FwdArgs& a,
                                        hipStream_t s);
// Chunk-partial region of the workspace (double2 x p.blocks).
double2* ws_partials(const Plan& p, void* ws);
// Tile groups of the depthwise forward (dw_conv.hip): tpp per plane, tiles_x
// across, each `rows` output rows (the last one clipped at Ho) by 64
// columns (the last tile of a row clipped at Wo).
struct DwStatsGeom {
    int64_t tpp = 0, tiles_x = 0, rows = 0;
};
// True when the forward runs the one-launch small-unit kernels (which take
// no partials from a producer).
bool forward_is_small(const Plan& p, const Tuning& t);
// The GroupNorm finish and apply from the depthwise forward's tile-group
// partials (`part`, dw_stats_geometry's layout) instead of chunk
// partials: mean / rstd / mean_lo, then y.  p: make_plan's plan for the
// output, whose workspace `a.ws` holds the rest.
hipError_t launch_forward_from_tile_partials(const Plan& p, const Tuning& t, const FwdArgs& a,
                                             const double2* part, const DwStatsGeom& g,
                                             int64_t Ho, int64_t Wo, hipStream_t s);
// Plan of the GroupNorm that follows a pointwise convolution: the chunk is
// the convolution's pixel chunk, so its epilogue partials are the plan's.
bool make_pw_plan(int64_t N, int64_t C_out, int64_t HW, int64_t G, const Tuning& t, Plan* p);

// Pointwise convolution (pw_conv.hip).
struct PwArgs {
    const float* x;     // [N][C_in][HW]
    const float* w;     // [C_out][C_in]
    const float* bias;  // [C_out], nullable
    float* z;           // [N][C_out][HW]
};
// C_in rounded up to a multiple of 8 (the kernel's K step).
int pw_kpad(int64_t C_in);
// The kernel addresses one sample's planes with 32-bit byte offsets.
bool pw_offsets_fit(int64_t C_in, int64_t HW);
// Pixels per wave of the pointwise convolution for this shape: at most
// max_chunk, a multiple of 128, small enough that about 2048 waves run.
int64_t pw_pick_chunk(int64_t N, int64_t C_out, int64_t HW, int64_t max_chunk);
// z = w * x + bias (z += w * x with `accumulate`).  With `part` non-null
// the kernel also writes the GroupNorm chunk partials of z for chunks of
// `chunk` pixels (a multiple of 128, normally from pw_pick_chunk),
// part[(n*C_out + co)*cpp + k].
// `name` labels the launch for the kernel timers (null: a default).
// Without `part`, the SIMT kernel (K split over the waves of a block) runs
// when pw_use_small(N, C_out, C_in, HW, small).  With `part` and `kz_ws`
// (at least pw_kz_bytes(N, C_out, HW, pw_kz_plan(...).kz) bytes, 16-byte
// aligned), a grid of few tiles splits K over up to kz_max blocks per tile
// (pw_kz_plan) and a second kernel adds their fp32 slices and writes the
// statistics (a 256 -> 128 output at 4096 pixels: 25.8 us with K over the
// four waves of a block, 14.3 + 4.5 us this way).
// `wt`: a.w holds the weights transposed, [C_in][C_out] (element (co, ci)
// at w[ci * C_out + co]); no bias, no statistics, no split over blocks.
hipError_t launch_pw_conv(const PwArgs& a, int64_t N, int64_t C_in, int64_t C_out,
                          int64_t HW, int64_t chunk, double2* part, bool accumulate,
                          int64_t small, float* kz_ws, int kz_max, hipStream_t s,
                          const char* name = nullptr, bool wt = false);
// Cross-block split-K of the MFMA convolution (kz = 1: not used).
struct PwKz {
    int kz = 1;
};
PwKz pw_kz_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t chunk,
                int kz_max);
size_t pw_kz_bytes(int64_t N, int64_t C_out, int64_t HW, int kz);
// Bound of pw_kz_bytes over every C_in (for workspace queries without it).
size_t pw_kz_max_bytes(int64_t N, int64_t C_out, int64_t HW, int64_t chunk, int kz_max);
// True when the SIMT kernel computes the M x HW outputs of N samples (K
// terms each): at most `small` multiply-adds, and offsets inside a sample
// fit in 32 bits.
bool pw_use_small(int64_t N, int64_t M, int64_t K, int64_t HW, int64_t small);

// Backward of the pointwise convolution: dx = W^T dz (written, or added
// with `accumulate_dx`), dw += sum dz x^T, db += sum dz; any output may be
// null.  Workspace: W^T, then the per-chunk dW and db partials.  The dx
// chunk is pw_pick_chunk(N, C_in, HW, chunk_dx).
struct PwBwdArgs {
    const float* dz;  // [N][C_out][HW]
    const float* x;   // [N][C_in][HW]
    const float* w;   // [C_out][C_in]
    float* dx;        // [N][C_in][HW], nullable
    float* dw;        // [C_out][C_in], nullable
    float* db;        // [C_out], nullable
    void* ws;
};
struct PwBwdPlan {
    int tm = 2, tn = 2;                  // 32-row MFMA tiles per dW tile (C_out, C_in)
    int64_t tiles_co = 0, tiles_ci = 0;  // (32 tm) x (32 tn) tiles of dW
    int64_t chunk = 0, cpp = 0, G = 0;   // pixel chunks of the dW waves
    int wpb = 1;                         // dW waves per block (1, 2, 4, 8)
    int64_t chunk_b = 0, cpp_b = 0, Gb = 0;  // their chunks: pixels, per plane, partials
    size_t wt_bytes = 0, pw_bytes = 0, pb_bytes = 0;
    int64_t chunk_dx = 0;  // pixels per wave of dx = W^T dz
    int kz_dx = 1;         // its cross-block split-K (pw_kz_plan)
    size_t kz_bytes = 0;   // and the slices' bytes, after the partials
};
PwBwdPlan make_pw_bwd_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW,
                           int64_t chunk_dx, int kz_max, int wg_waves, int64_t wg_target);
size_t pw_bwd_workspace_bytes(const PwBwdPlan& p);
// dx runs the SIMT kernel when pw_use_small(N, C_in, C_out, HW, small),
// dW/db when the weight gradient has at most small/2 multiply-adds and
// N*HW <= 16384 (then the workspace is not touched).  `chunk_dx` and the
// split-K of dx come from the plan (make_pw_bwd_plan).
hipError_t launch_pw_backward(const PwBwdPlan& p, const PwBwdArgs& a, int64_t N, int64_t C_in,
                              int64_t C_out, int64_t HW, bool accumulate_dx, int64_t small,
                              hipStream_t s);

// Fused backward of a pointwise CBA block (pw_conv.hip): from the
// GroupNorm input z, the upstream gradient dy and the convolution input x,
// dx (=, or += with accumulate_dx) W^T dz and dw += sum dz x^T with dz the
// GroupNorm(+SiLU) input gradient, never stored.  C_in, C_out multiples of 8
// up to 64, HW % 4 == 0, 16-byte aligned tensors (pw_cba_fused_fits).  The GroupNorm sums
// come from launch_backward_sums; block 0 also adds dgamma / dbeta.
struct PwCbaArgs {
    const float* dy;  // [N][C_out][HW]
    const float* z;   // [N][C_out][HW], the GroupNorm input
    const float* x;   // [N][C_in][HW], the convolution input
    const float* w;   // [C_out][C_in]
    const float* gamma;
    const float* beta;
    const float* mean;
    const float* rstd;
    const float* mean_lo;
    const double2* unit_sums;
    const double2* plane_sums;
    float* dgamma;  // nullable
    float* dbeta;   // nullable
    float* dx;      // nullable
    float* dw;      // nullable
    float* part_w;  // [blocks][C_out][C_in] workspace (with dw)
    // unit_sums and plane_sums null: the GroupNorm reduction's chunk
    // partials, cpp per plane, whose finish each block folds
    const double2* gn_part = nullptr;
    int64_t gn_cpp = 0;
};
struct PwCbaPlan {
    int64_t chunk = 0, cpp = 0, blocks = 0;  // pixels per block, per plane, all
    size_t part_bytes = 0;                   // dW partials
};
bool pw_cba_fused_fits(int64_t C_in, int64_t C_out, int64_t HW);
// About `target` blocks of 4 waves (a chunk of at least 128 pixels).
PwCbaPlan make_pw_cba_plan(int64_t N, int64_t C_in, int64_t C_out, int64_t HW, int64_t target);
hipError_t launch_pw_cba_backward(const PwCbaPlan& p, const PwCbaArgs& a, int64_t N,
                                  int64_t C_in, int64_t C_out, int64_t HW, int64_t G, bool silu,
                                  bool accumulate_dx, hipStream_t s);

// Depthwise convolution (dw_conv.hip): groups = C_in = C_out, weights
// [C][K][K], output size given by the caller, taps outside the input skipped.
struct DwShape {
    int64_t N = 0, C = 0, Hi = 0, Wi = 0, Ho = 0, Wo = 0;
    int64_t K = 0, pad = 0, S = 1, D = 1;
};
// True if (K, S, D) has a tiled kernel (else the generic kernels run).
bool dw_has_fast(int64_t K, int64_t S, int64_t D);
// Workspace of the backward (per-tile weight-gradient partials).
size_t dw_bwd_workspace_bytes(const DwShape& sh);
// Blocks of the tiled kernels over the output (or, for dx, input) planes.
int64_t dw_grid_blocks(const DwShape& sh, bool output_tiles);
// With `part` (a shape with a tiled kernel, dw_stats_geometry true), the
// forward also writes the GroupNorm chunk partials of y: part[plane * tpp
// + group] = (mean, M2) of the group's outputs.
hipError_t launch_dw_forward(const DwShape& sh, const float* x, const float* w,
                             const float* bias, float* y, hipStream_t s,
                             double2* part = nullptr);
// Tile groups of the forward (DwStatsGeom); false if the shape has no
// tiled forward.
bool dw_stats_geometry(const DwShape& sh, DwStatsGeom* g);
// dx (+)= input gradient, dw += weight gradient, db += bias gradient; any
// output may be null.
hipError_t launch_dw_backward(const DwShape& sh, const float* dy, const float* x,
                              const float* w, float* dx, float* dw, float* db,
                              bool accumulate_dx, void* ws, hipStream_t s);

// Fused backward of a depthwise CBA block with a stride-1 "same"
// convolution (dw_conv.hip): from z (the GroupNorm input), dy and x, dx
// (=, or += with accumulate_dx) flip(w) (*) dz and dw += the weight
// gradient, with dz the GroupNorm(+SiLU) input gradient formed in LDS and
// never stored.  The GroupNorm sums come from launch_backward_sums; the
// kernel also adds dgamma / dbeta.  Needs dw_cba_fused_fits and, with dw,
// dw_cba_part_bytes of workspace at `part`.
struct DwCbaArgs {
    const float* dy;  // [N][C][H][W]
    const float* z;
    const float* x;
    const float* w;  // [C][K][K]
    const float* gamma;
    const float* beta;
    const float* mean;
    const float* rstd;
    const float* mean_lo;
    const double2* unit_sums;
    const double2* plane_sums;
    float* dgamma;  // nullable
    float* dbeta;   // nullable
    float* dx;      // [N][C][H][W]
    float* dw;      // [C][K][K], nullable
    float* part;    // weight-gradient block partials
    // unit_sums and plane_sums null: the GroupNorm reduction's chunk
    // partials, cpp per plane, whose finish each block folds (C / G at most
    // kFoldPlanes)
    const double2* gn_part = nullptr;
    int64_t gn_cpp = 0;
};
bool dw_cba_fused_fits(const DwShape& sh);
size_t dw_cba_part_bytes(const DwShape& sh);
int64_t dw_cba_grid_blocks(const DwShape& sh);
hipError_t launch_dw_cba_backward(const DwShape& sh, const DwCbaArgs& a, int64_t G, bool silu,
                                  bool accumulate_dx, hipStream_t s);

// Elementwise kernels (elementwise.hip).
hipError_t launch_silu_forward(const float* x, float* y, int64_t n,
                               hipStream_t s);
hipError_t launch_silu_backward(const float* gy, const float* x, float* gx,
                                int64_t n, hipStream_t s);
hipError_t launch_add_forward(const float* a, const float* b, float* y,
                              int64_t n, hipStream_t s);
hipError_t launch_add_backward(const float* gy, float* ga, float* gb,
                               int64_t n, hipStream_t s);
hipError_t launch_fill(float* p, float v, int64_t n, hipStream_t s);

// Deferred weight-gradient finishes (wfinish.hip).  An entry adds
// sum_g part[g][e] (float64, k_sum_partials' order) into out0[e] (kk1 = 0)
// or, for the depthwise layout e = c*kk1 + k, into tap c*(kk1-1) + k of
// out0 (k < kk1 - 1) or bias c of out1 (k = kk1 - 1); null outputs skip.
struct WeightFinish {
    const float* part;  // [G][E] fp32 partials
    float* out0;
    float* out1;
    int64_t E, G, kk1;
};
// While a C-ABI call with SOAR_DEFER_WEIGHT_FINISH runs, its launchers
// queue their finishes on the calling thread (weight_finish_queue returns
// true; *err reports a flush the queue had to run first: a finish on
// another stream, or one adding into weights already queued) instead of
// launching them; weight_finish_flush launches everything queued, on the
// stream it was queued on.
void weight_finish_defer(bool on);
bool weight_finish_deferring();
bool weight_finish_queue(const WeightFinish& f, hipStream_t s, hipError_t* err);
hipError_t weight_finish_flush();
// Called by a convolution backward entry point before it launches anything:
// flushes the queue when its weight gradients [o0, o0 + n0) and
// [o1, o1 + n1) overlap a queued finish's (whatever `defer`: the additions
// keep their call order) or when a deferring call comes on another stream.
hipError_t weight_finish_before(const float* o0, int64_t n0, const float* o1, int64_t n1,
                                hipStream_t s, bool defer);
size_t weight_finish_pending();
hipStream_t weight_finish_stream();
void weight_finish_discard();

// Kernel timing hooks (capi.cpp).  prof_begin returns a token passed to
// prof_end; both are no-ops while timing is off.
int prof_begin(hipStream_t s, const char* kernel);
void prof_end(hipStream_t s, int token);

// sum_{g0 <= g < g1} part[g * E + e] in float64, g ascending: full batches
// of eight loads with no bounds test between them (a test per load makes
// the compiler wait for each one), then the tail.  (Batches of 32, with the
// tail in one batch, measured slower in the finish kernels.)
__device__ __forceinline__ double segment_sum(const float* __restrict__ part, int64_t E,
                                              int64_t e, int64_t g0, int64_t g1) {
    constexpr int kU = 8;
    double sum = 0.0;
    int64_t gg = g0;
    for (; gg + kU <= g1; gg += kU) {
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = part[(gg + u) * E + e];
#pragma unroll
        for (int u = 0; u < kU; ++u) sum += (double)v[u];
    }
    for (; gg < g1; ++gg) sum += (double)part[gg * E + e];
    return sum;
}

}  // namespace gn
}  // namespace soar
