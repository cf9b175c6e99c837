"""Benchmark of the MI355X GroupNorm+SiLU path (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one forward + backward of fused GroupNorm+SiLU at BASELINE
config 3 (N=1, C=64, H=W=2048, G=16, fp32), inputs resident in HBM, run
through the C-ABI of libsoar_gn.so on one GPU.  Prints one JSON line:

  value      algorithmic HBM bytes of the step (8 tensor passes: fwd 3T,
             bwd 5T, T = N*C*H*W*4) / measured step time, in GB/s;
  roofline   the dominant kernel's algorithmic bytes per launch / its mean
             hipEvent-timed duration over the timed region, against the
             8 TB/s HBM peak; `traffic` is the rocprofv3-measured bytes per
             launch from profiles/ when present;
  cpu_baseline  the fp32 statement of the reference's CPU loops
             (oracle/soar_oracle.c, one pinned core, median of 3) on a
             bounded sample of config 3, plus config 1 at full size.

Other workloads (--config): the other BASELINE configs (cfg1_fwd, cfg2_fwd,
cfg4_chain, cfg5), the CBA block with a pointwise conv (cba_pw), the CBA
depthwise convolutions at 1x64x2048^2 (dw_k3, dw_k5, dw_k7, dw_k3d5,
dw_k3s2), SOAR training steps (train_nano64/512/1024), SOAR predictions
(predict_nano64/1024) and the streaming
ceilings of this memory system for plain kernels of the library's shape
(stream_read, stream_copy, stream_2r1w, stream_2r over 1 GiB buffers; stream_planes_read,
stream_planes_copy, stream_planes_copy_pad4k: the pointwise convolution's 64-plane pattern).
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "soar.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "GN+SiLU fwd+bwd achieved HBM GB/s (% of peak), 1×64×2048² fp32"
PEAK_GBS = 8000.0
SEED = 20261201

CONFIGS = {
    # name: (N, C, HW, G, passes, residual, blocks)
    "cfg1_fwd": (1, 32, 256 * 256, 8, "fwd", False, 1),
    "cfg2_fwd": (1, 32, 2048 * 2048, 8, "fwd", False, 1),
    "cfg3": (1, 64, 2048 * 2048, 16, "fwdbwd", False, 1),
    "cfg4_chain": (2, 128, 1024 * 1024, 32, "fwdbwd", True, 6),
    "cfg5": (1, 16, 2048 * 2048, 4, "fwdbwd", False, 1),
    # CBA block with a pointwise conv (64 -> 64 channels) feeding config 3's
    # GroupNorm+SiLU; C is C_out, the conv's C_in is CBA_C_IN
    "cba_pw": (1, 64, 2048 * 2048, 16, "fwdbwd", False, 1),
    "cba_pw_unfused": (1, 64, 2048 * 2048, 16, "fwdbwd", False, 1),
}
SEED_OF = {"cfg1_fwd": SEED + 1, "cfg2_fwd": SEED + 2, "cfg3": SEED + 3, "cfg4_chain": SEED + 4, "cfg5": SEED + 5,
           "cba_pw": SEED + 6, "cba_pw_unfused": SEED + 6}
CBA_C_IN = 64
PEAK_MFMA_F32 = 157.3  # TFLOP/s, dense fp32 matrix

# Streaming ceilings (libsoar_synth.so soar_synth_stream over 1 GiB
# buffers): name -> pattern
STREAM_CONFIGS = {"stream_read": "read", "stream_copy": "copy", "stream_2r1w": "2r1w",
                  "stream_2r": "2r",
                  # the pointwise convolution's access pattern over 64 planes of
                  # 16 MiB (a 1 GiB NCHW tensor), at the tensor's plane stride and
                  # with the stride padded by 4 KiB
                  "stream_planes_read": "planes_read", "stream_planes_copy": "planes_copy",
                  "stream_planes_copy_pad4k": "planes_copy_pad",
                  # all four patterns in several launch shapes + the runtime's D2D copy
                  "stream_sweep": "sweep"}

# Depthwise convolutions of the CBA blocks at 1x64x2048^2, forward + backward
# (dx, dW, db): name -> (K, stride, dilation); pad = dilation*(K-1)/2
DW_CONFIGS = {"dw_k3": (3, 1, 1), "dw_k5": (5, 1, 1), "dw_k7": (7, 1, 1),
              "dw_k3d5": (3, 1, 5), "dw_k3s2": (3, 2, 1)}
DW_SHAPE = (1, 64, 2048, 2048)
# CBA blocks with a depthwise conv (stride 1, same padding) at 1x64x2048^2,
# G = 16, forward + backward; the backward fused (soar_dw_cba_backward) or
# as the GroupNorm backward then the depthwise backward: name -> (K, dil)
CBA_DW_CONFIGS = {}
for _k, _d in ((3, 1), (5, 1), (7, 1), (3, 5)):
    _n = f"cba_dw_k{_k}" + (f"d{_d}" if _d > 1 else "")
    CBA_DW_CONFIGS[_n] = (_k, _d, True)
    CBA_DW_CONFIGS[_n + "_unfused"] = (_k, _d, False)
PEAK_VALU_F32 = 157.3  # TFLOP/s, MI355X published vector fp32 (packed); 78.6 without

# End-to-end training steps of the SOAR model through libsoar_host.so
# (soar_train_step: forward, Dice+BCE loss, backward, clip, AdamW), one
# 1-channel image per step: name -> (variant, H, W)
TRAIN_CONFIGS = {
    "train_nano64": ("nano", 64, 64),
    "train_nano512": ("nano", 512, 512),
    "train_nano1024": ("nano", 1024, 1024),
}
# soar_predict of the same model: no-grad forward, sigmoid, threshold,
# probabilities, mask and RLE back to the host
PREDICT_CONFIGS = {
    "predict_nano64": ("nano", 64, 64),
    "predict_nano1024": ("nano", 1024, 1024),
}

# algorithmic tensor passes (units of T) each kernel makes per block of the
# step, summed over its launches (a kernel runs once per unit batch)
PASSES = {"gn_stats_partial": 1, "gn_silu_apply": 2, "gn_silu_bwd_reduce": 2,
          "gn_silu_bwd_dx": 3, "gn_stats_finish": 0, "gn_bwd_finish": 0,
          "gn_param_finish": 0}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg3",
                    choices=sorted(CONFIGS) + sorted(TRAIN_CONFIGS) + sorted(PREDICT_CONFIGS)
                    + sorted(STREAM_CONFIGS)
                    + sorted(DW_CONFIGS) + sorted(CBA_DW_CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="time the steps without per-kernel events")
    ap.add_argument("--no-eager", action="store_true",
                    help="train configs: skip the second, graph-off handle (for tracing)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a plain 1 GiB copy kernel (for rocprofv3 counter scaling)")
    ap.add_argument("--tune", action="append", default=[], metavar="NAME=VALUE",
                    help="set a library tuning key before the run (soar_gn_tune; NAME is a "
                         "TUNE_* name of soar_gn.py without the prefix, e.g. NT_LOAD=3); "
                         "repeatable, recorded in the JSON line's config")
    return ap.parse_args()


def apply_tuning(args):
    """Sets the --tune keys; returns {name: value} for the JSON line."""
    if not args.tune:
        return {}
    import soar_gn as gn
    out = {}
    for item in args.tune:
        name, _, value = item.partition("=")
        key = getattr(gn, "TUNE_" + name.strip().upper(), None)
        if key is None or not value:
            sys.exit(f"--tune {item!r}: expected NAME=VALUE with NAME a soar_gn TUNE_* key")
        gn.tune(key, int(value))
        out[name.strip().upper()] = int(value)
    return out


def traffic_from_profiles(config):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 PMC summary (a `TRAFFIC_JSON:` line), else None."""
    path = os.path.join(ROOT, "profiles", f"pmc_{config}.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            m = re.match(r"\s*TRAFFIC_JSON:\s*(\{.*\})", line)
            if m:
                return json.loads(m.group(1))
    return None


def make_inputs(gn, N, C, HW, G, seed, blocks):
    import torch
    x = torch.empty((N, C, HW), device="cuda")
    dy = torch.empty_like(x)
    gn.synth_normal(x, seed, 1, 0.0, 1.0)
    gn.synth_normal(dy, seed, 4, 0.0, 1e-2)
    params = []
    for b in range(blocks):
        gamma = torch.empty(C, device="cuda")
        beta = torch.empty(C, device="cuda")
        gn.synth_uniform(gamma, seed + 1000 * b, 2, 0.5, 1.5)
        gn.synth_normal(beta, seed + 1000 * b, 3, 0.0, 0.1)
        params.append((gamma, beta))
    return x, dy, params


class Step:
    """Preallocated buffers and the launch sequence of one step."""

    def __init__(self, gn, N, C, HW, G, passes, residual, blocks, seed):
        import torch
        self.gn, self.G, self.passes, self.residual = gn, G, passes, residual
        self.x, self.dy, self.params = make_inputs(gn, N, C, HW, G, seed, blocks)
        # activations of a chain: acts[0] = input, acts[b+1] = block b output
        self.acts = [self.x] + [torch.empty_like(self.x) for _ in range(blocks)]
        self.mean = [torch.empty(N * G, device="cuda") for _ in range(blocks)]
        self.rstd = [torch.empty(N * G, device="cuda") for _ in range(blocks)]
        self.mean_lo = [torch.empty(N * G, device="cuda") for _ in range(blocks)]
        self.ws = gn.workspace(N, C, HW, G)
        self.grads = [torch.empty_like(self.x) for _ in range(2)] if passes == "fwdbwd" else []
        self.dparams = [(torch.zeros(C, device="cuda"), torch.zeros(C, device="cuda"))
                        for _ in range(blocks)]
        self.T = N * C * HW * 4

    def algorithmic_bytes(self):
        per_block = 3 if self.passes == "fwd" else 8
        return per_block * len(self.params) * self.T

    def __call__(self):
        gn = self.gn
        for b, (gamma, beta) in enumerate(self.params):
            gn.gn_silu_forward(self.acts[b], gamma, beta, self.G, eps=1e-5,
                               residual=self.residual, y=self.acts[b + 1], mean=self.mean[b],
                               rstd=self.rstd[b], mean_lo=self.mean_lo[b], ws=self.ws)
        if self.passes == "fwd":
            return
        g_in = self.dy
        for b in reversed(range(len(self.params))):
            gamma, beta = self.params[b]
            g_out = self.grads[b % 2]
            dg, db = self.dparams[b]
            gn.gn_silu_backward(g_in, self.acts[b], gamma, beta,
                                (self.mean[b], self.rstd[b], self.mean_lo[b]), self.G, residual=self.residual, dx=g_out, dgamma=dg, dbeta=db,
                                ws=self.ws)
            g_in = g_out


class CBAStep:
    """Forward and backward of a CBA block whose conv is pointwise:
    z = conv1x1(x), y = SiLU(GroupNorm(z)) with the GroupNorm statistics in
    the conv epilogue (soar_pw_conv_gn_silu_forward).  Backward, fused
    (cba_pw): soar_pw_cba_backward, the GroupNorm reduction over (z, dy) and
    then one kernel that forms dz in registers and computes dx and dW from
    it.  Unfused (cba_pw_unfused): soar_gn_silu_backward (dy -> dz, dgamma,
    dbeta) then soar_pw_conv_backward (dz -> dx, dW)."""

    def __init__(self, gn, N, C, HW, G, seed, fused=True):
        import torch
        self.gn, self.G, self.fused = gn, G, fused
        self.C_in, self.C_out, self.N, self.HW = CBA_C_IN, C, N, HW
        self.x = torch.empty((N, self.C_in, HW), device="cuda")
        gn.synth_normal(self.x, seed, 1, 0.0, 1.0)
        self.w = torch.empty((C, self.C_in), device="cuda")
        gn.synth_uniform(self.w, seed, 7, -self.C_in ** -0.5, self.C_in ** -0.5)
        self.gamma = torch.empty(C, device="cuda")
        self.beta = torch.empty(C, device="cuda")
        gn.synth_uniform(self.gamma, seed, 2, 0.5, 1.5)
        gn.synth_normal(self.beta, seed, 3, 0.0, 0.1)
        self.z = torch.empty((N, C, HW), device="cuda")
        self.y = torch.empty_like(self.z)
        self.mean = torch.empty(N * G, device="cuda")
        self.rstd = torch.empty(N * G, device="cuda")
        self.mean_lo = torch.empty(N * G, device="cuda")
        self.ws = torch.empty(gn.pw_conv_gn_workspace_bytes(N, C, HW, G), dtype=torch.uint8,
                              device="cuda")
        self.dy = torch.empty((N, C, HW), device="cuda")
        gn.synth_normal(self.dy, seed, 4, 0.0, 1e-2)
        self.dz = torch.empty_like(self.z)
        self.dx = torch.empty_like(self.x)
        self.dw = torch.zeros_like(self.w)
        self.dgamma = torch.zeros(C, device="cuda")
        self.dbeta = torch.zeros(C, device="cuda")
        self.ws_gn = gn.workspace(N, C, HW, G)
        if fused:
            self.ws_bwd = torch.empty(gn.pw_cba_backward_workspace_bytes(N, self.C_in, C, HW, G),
                                      dtype=torch.uint8, device="cuda")
        else:
            self.ws_bwd = torch.empty(gn.pw_conv_backward_workspace_bytes(N, self.C_in, C, HW),
                                      dtype=torch.uint8, device="cuda")
        self.params = [None]
        self.T = N * C * HW * 4

    def algorithmic_bytes(self):
        # fwd: conv reads x, writes z; apply reads z, writes y.
        # bwd fused: GN reduce reads dy, z; the fused kernel reads dy, z, x
        # and writes dx.  Unfused: GN reduce reads dy, z; GN dx reads dy, z,
        # writes dz; conv dx reads dz, writes dx; conv dW reads dz, x.
        # (Weights are noise.)
        ti, to = self.C_in, self.C_out
        bwd = 4 * to + 2 * ti if self.fused else 7 * to + 2 * ti
        return (ti + 3 * to + bwd) * self.N * self.HW * 4

    def kernel_bytes(self, name):
        nb = self.N * self.HW * 4
        ti, to = self.C_in * nb, self.C_out * nb
        return {"pw_conv_gn_stats": ti + to, "gn_silu_apply": 2 * to,
                "gn_silu_bwd_reduce": 2 * to, "gn_silu_bwd_dx": 3 * to,
                "pw_conv_dgrad": to + ti, "pw_conv_wgrad": to + ti,
                "pw_cba_bwd": 2 * to + 2 * ti}.get(name, 0)

    def kernel_flops(self, name):
        f = 2 * self.C_in * self.C_out * self.N * self.HW
        if name == "pw_cba_bwd":
            return 2 * f  # dx and dW
        return f if name in ("pw_conv_gn_stats", "pw_conv_dgrad", "pw_conv_wgrad") else 0

    def __call__(self):
        gn = self.gn
        gn.pw_conv_gn_silu_forward(self.x, self.w, None, self.gamma, self.beta, self.G,
                                   eps=1e-5, z=self.z, y=self.y, mean=self.mean, rstd=self.rstd,
                                   mean_lo=self.mean_lo, ws=self.ws)
        st = gn.Stats(self.mean, self.rstd, self.mean_lo)
        if self.fused:
            gn.pw_cba_backward(self.dy, self.z, self.x, self.w, self.gamma, self.beta, st, self.G,
                               dx=self.dx, dweight=self.dw, dgamma=self.dgamma,
                               dbeta=self.dbeta, ws=self.ws_bwd)
            return
        gn.gn_silu_backward(self.dy, self.z, self.gamma, self.beta, st, self.G, dx=self.dz,
                            dgamma=self.dgamma, dbeta=self.dbeta, ws=self.ws_gn)
        gn.pw_conv_backward(self.dz, self.x, self.w, dx=self.dx, dweight=self.dw, want_db=False,
                            ws=self.ws_bwd)


class DwStep:
    """Forward and backward (dx, dW, db) of one depthwise convolution of the
    CBA blocks at 1x64x2048^2 (soar_dw_conv_forward / soar_dw_conv_backward):
    LKR's k5 / k7, Ctx's dilated k3, Down's stride-2 k3."""

    def __init__(self, gn, name, seed):
        import torch
        K, S, D = DW_CONFIGS[name]
        N, C, H, W = DW_SHAPE
        self.gn, self.K, self.S, self.D, self.pad = gn, K, S, D, D * (K - 1) // 2
        self.N, self.C, self.H, self.W = N, C, H, W
        self.Ho = gn.conv_out_size(H, K, self.pad, S, D)
        self.Wo = gn.conv_out_size(W, K, self.pad, S, D)
        self.x = torch.empty((N, C, H, W), device="cuda")
        gn.synth_normal(self.x, seed, 1, 0.0, 1.0)
        self.w = torch.empty((C, K, K), device="cuda")
        gn.synth_uniform(self.w, seed, 7, -1.0 / K, 1.0 / K)
        self.b = torch.empty(C, device="cuda")
        gn.synth_normal(self.b, seed, 3, 0.0, 0.1)
        self.y = torch.empty((N, C, self.Ho, self.Wo), device="cuda")
        self.dy = torch.empty_like(self.y)
        gn.synth_normal(self.dy, seed, 4, 0.0, 1e-2)
        self.dx = torch.empty_like(self.x)
        self.dw = torch.zeros_like(self.w)
        self.db = torch.zeros_like(self.b)
        nws = int(gn.lib().soar_dw_conv_backward_workspace_bytes(N, C, H, W, self.Ho, self.Wo,
                                                                 K, S, D))
        self.ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
        self.params = [None]
        self.T_in = N * C * H * W * 4
        self.T_out = N * C * self.Ho * self.Wo * 4

    def algorithmic_bytes(self):
        # fwd reads x, writes y; dgrad reads dy, writes dx; wgrad reads dy, x
        return 3 * (self.T_in + self.T_out)

    def kernel_bytes(self, name):
        return {"dw_conv": self.T_in + self.T_out, "dw_conv_dgrad": self.T_in + self.T_out,
                "dw_conv_wgrad": self.T_in + self.T_out}.get(name, 0)

    def kernel_flops(self, name):
        f = 2 * self.K * self.K * self.T_out // 4
        return f if name in ("dw_conv", "dw_conv_dgrad", "dw_conv_wgrad") else 0

    def config(self):
        return {"workload": f"depthwise conv k{self.K} stride {self.S} dilation {self.D} pad "
                            f"{self.pad}, fwd + bwd (dx, dW, db)",
                "N": self.N, "C": self.C, "H": self.H, "W": self.W, "H_out": self.Ho,
                "W_out": self.Wo}

    def __call__(self):
        gn = self.gn
        gn.dw_conv_forward(self.x, self.w, self.b, self.pad, self.S, self.D, y=self.y)
        gn.dw_conv_backward(self.dy, self.x, self.w, self.pad, self.S, self.D, dx=self.dx,
                            dweight=self.dw, dbias=self.db, ws=self.ws)


class CBADwStep:
    """Forward and backward of a CBA block with a depthwise conv (stride 1,
    same padding, no bias) at 1x64x2048^2, G = 16.  Fused: the forward
    soar_dw_conv_gn_silu_forward (the GroupNorm statistics in the
    convolution's epilogue, then the finish and apply) and the backward
    soar_dw_cba_backward (the GroupNorm reduction, then one kernel that forms
    dz per tile in LDS and computes dx and dW from it).  Unfused: z =
    dwconv(x) (soar_dw_conv_forward), y = SiLU(GroupNorm(z))
    (soar_gn_silu_forward); soar_gn_silu_backward to dz, then
    soar_dw_conv_backward."""

    def __init__(self, gn, name, seed):
        import torch
        K, D, fused = CBA_DW_CONFIGS[name]
        N, C, H, W = DW_SHAPE
        self.gn, self.K, self.D, self.pad, self.fused = gn, K, D, D * (K - 1) // 2, fused
        self.N, self.C, self.H, self.W, self.G = N, C, H, W, 16
        self.x = torch.empty((N, C, H, W), device="cuda")
        gn.synth_normal(self.x, seed, 1, 0.0, 1.0)
        self.w = torch.empty((C, K, K), device="cuda")
        gn.synth_uniform(self.w, seed, 7, -1.0 / K, 1.0 / K)
        self.gamma = torch.empty(C, device="cuda")
        self.beta = torch.empty(C, device="cuda")
        gn.synth_uniform(self.gamma, seed, 2, 0.5, 1.5)
        gn.synth_normal(self.beta, seed, 3, 0.0, 0.1)
        self.z, self.y = torch.empty_like(self.x), torch.empty_like(self.x)
        self.dy = torch.empty_like(self.x)
        gn.synth_normal(self.dy, seed, 4, 0.0, 1e-2)
        self.mean, self.rstd, self.lo = (torch.empty(N * self.G, device="cuda") for _ in range(3))
        self.dx, self.dz = torch.empty_like(self.x), torch.empty_like(self.x)
        self.dw = torch.zeros_like(self.w)
        self.dgamma, self.dbeta = torch.zeros(C, device="cuda"), torch.zeros(C, device="cuda")
        self.ws_gn = gn.workspace(N, C, H * W, self.G)
        self.ws_fwd = torch.empty(
            max(gn.dw_conv_gn_workspace_bytes(N, C, H, W, H, W, K, self.pad, 1, D, self.G), 1),
            dtype=torch.uint8, device="cuda")
        if fused:
            nws = gn.dw_cba_backward_workspace_bytes(N, C, H, W, H, W, K, self.pad, 1, D, self.G)
        else:
            nws = int(gn.lib().soar_dw_conv_backward_workspace_bytes(N, C, H, W, H, W, K, 1, D))
        self.ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
        self.params = [None]
        self.T = N * C * H * W * 4

    def algorithmic_bytes(self):
        # fwd: conv reads x, writes z (fused: with the GroupNorm statistics);
        # unfused, the statistics read z again; apply reads z, writes y.  bwd:
        # the reduction reads dy, z; fused: one kernel reads dy, z, x and
        # writes dx; unfused: GroupNorm dx reads dy, z and writes dz, dgrad
        # reads dz and writes dx, wgrad reads dz and x.
        return ((4 + 2 + 4) if self.fused else (5 + 2 + 7)) * self.T

    def kernel_bytes(self, name):
        T = self.T
        return {"dw_conv": 2 * T, "dw_conv_stats": 2 * T, "gn_stats_partial": T,
                "gn_silu_apply": 2 * T,
                "gn_silu_bwd_reduce": 2 * T, "gn_silu_bwd_dx": 3 * T, "dw_conv_dgrad": 2 * T,
                "dw_conv_wgrad": 2 * T, "dw_cba_bwd": 4 * T}.get(name, 0)

    def kernel_flops(self, name):
        f = 2 * self.K * self.K * self.T // 4
        if name == "dw_cba_bwd":
            return 2 * f
        return f if name in ("dw_conv", "dw_conv_stats", "dw_conv_dgrad", "dw_conv_wgrad") else 0

    def config(self):
        return {"workload": f"CBA fwd+bwd: depthwise conv k{self.K} dilation {self.D} pad "
                            f"{self.pad} + GN + SiLU, "
                            + ("GN statistics in the conv epilogue, backward fused (dz per tile "
                               "in LDS)" if self.fused else
                               "conv then GN forward, backward as GN backward then depthwise "
                               "backward"),
                "N": self.N, "C": self.C, "H": self.H, "W": self.W, "G": self.G}

    def __call__(self):
        gn = self.gn
        if self.fused:
            gn.dw_conv_gn_silu_forward(self.x, self.w, None, self.gamma, self.beta, self.G,
                                       self.pad, 1, self.D, z=self.z, y=self.y, mean=self.mean,
                                       rstd=self.rstd, mean_lo=self.lo, ws=self.ws_fwd)
        else:
            gn.dw_conv_forward(self.x, self.w, None, self.pad, 1, self.D, y=self.z)
            gn.gn_silu_forward(self.z, self.gamma, self.beta, self.G, y=self.y, mean=self.mean,
                               rstd=self.rstd, mean_lo=self.lo, ws=self.ws_gn)
        st = gn.Stats(self.mean, self.rstd, self.lo)
        if self.fused:
            gn.dw_cba_backward(self.dy, self.z, self.x, self.w, self.gamma, self.beta, st, self.G,
                               self.pad, 1, self.D, dx=self.dx, dweight=self.dw,
                               dgamma=self.dgamma, dbeta=self.dbeta, ws=self.ws)
            return
        gn.gn_silu_backward(self.dy, self.z, self.gamma, self.beta, st, self.G, dx=self.dz,
                            dgamma=self.dgamma, dbeta=self.dbeta, ws=self.ws_gn)
        gn.dw_conv_backward(self.dz, self.x, self.w, self.pad, 1, self.D, dx=self.dx,
                            dweight=self.dw, want_db=False, ws=self.ws)


# Other launch shapes of the four streaming patterns (libsoar_synth.so
# soar_synth_stream_shape) and the runtime's D2D copy, over the same 1 GiB
# buffers: is the library's shape or the memory system the ceiling?
# (label, threads, loads in flight, chunk floats or None, persistent grid or
# None, non-temporal loads)
SWEEP_SHAPES = [
    ("chunk 256 thr x 4 loads, 8192 floats, nt loads", 256, 4, 8192, None, True),
    ("chunk 512 thr x 2 loads, 4096 floats", 512, 2, 4096, None, False),
    ("chunk 1024 thr x 4 loads, 32768 floats", 1024, 4, 32768, None, False),
    ("chunk 1024 thr x 4 loads, 32768 floats, nt loads", 1024, 4, 32768, None, True),
    ("persistent 4 blocks/CU x 256 thr x 8 loads, nt loads", 256, 8, None, 1024, True),
    ("persistent 2 blocks/CU x 1024 thr x 8 loads", 1024, 8, None, 512, False),
]


def bench_stream_sweep(args):
    """Every streaming pattern in the library's shape (k_stream), in the
    SWEEP_SHAPES, and the copy through hipMemcpyAsync D2D: median of the
    launches between hipEvents, GB/s of the pattern's tensor bytes.
    value = the best copy (1R1W) rate found."""
    import torch
    import soar_gn as gn
    n = 1 << 28
    a = torch.empty(n, device="cuda")
    b = torch.empty(n, device="cuda")
    out = torch.empty(n, device="cuda")
    gn.synth_normal(a, SEED, 1)
    gn.synth_normal(b, SEED, 4)
    gn.synth_normal(out, SEED, 2)

    def time_it(launch):
        for _ in range(args.warmup):
            launch()
        torch.cuda.synchronize()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.steps)]
        for e0, e1 in evs:
            e0.record()
            launch()
            e1.record()
        torch.cuda.synchronize()
        ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
        return ms[len(ms) // 2]

    results = {}
    t0 = time.perf_counter()
    for pattern in ("read", "copy", "2r1w", "2r"):
        passes = gn.STREAM_KINDS[pattern][1]
        rows = {}

        def add(label, launch):
            ms = time_it(launch)
            rows[label] = {"ms": round(ms, 4), "GBps": round(passes * n * 4 / (ms * 1e-3) / 1e9, 1)}

        add("library shape: chunk 256 thr x 4 loads, 8192 floats (k_stream)",
            lambda: gn.synth_stream(pattern, a, b, out))
        for label, thr, loads, chunk, grid, ntl in SWEEP_SHAPES:
            add(label, lambda: gn.synth_stream_shape(pattern, a, b, out, thr, loads, chunk=chunk,
                                                     grid=grid, ntl=ntl))
        if pattern == "copy":
            add("runtime hipMemcpyAsync D2D", lambda: gn.synth_memcpy_d2d(out, a))
        results[pattern] = rows
    wall = time.perf_counter() - t0
    best = {p: max(r.values(), key=lambda v: v["GBps"]) for p, r in results.items()}
    value = best["copy"]["GBps"]
    print(json.dumps({
        "metric": "stream_sweep: best copy (1R1W) GB/s over 1 GiB buffers, across launch shapes",
        "value": value, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": best["copy"]["ms"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic N(0,1)",
        "config": {"workload": "streaming patterns read / copy / 2r1w / 2r in several launch "
                               "shapes and the runtime's D2D copy, 1 GiB buffers"},
        "frac_of_peak": round(value / PEAK_GBS, 4), "wall_s_timed": round(wall, 4),
        "best": {p: v["GBps"] for p, v in best.items()}, "shapes": results}), flush=True)


def bench_stream(args):
    """Streaming ceilings: one synth_stream kernel over 1 GiB buffers, each
    launch between hipEvents on the launch stream; value = tensor bytes of
    the pattern / median launch time."""
    import torch
    import soar_gn as gn
    pattern = STREAM_CONFIGS[args.config]
    n = 1 << 28
    if pattern.startswith("planes"):
        plane = n // 64
        stride = plane + (1024 if pattern.endswith("pad") else 0)
        a = torch.empty(64 * stride, device="cuda")
        out = torch.empty(64 * stride, device="cuda")
        gn.synth_normal(a, SEED, 1)
        write = pattern != "planes_read"
        passes = 2 if write else 1
        kname = f"k_planes<{str(write).lower()}>"
        launch = lambda: gn.synth_planes(write, a, out, plane, stride)
        what = (f"the pointwise convolution's pattern over 64 planes of 16 MiB, plane stride "
                f"{stride * 4} bytes: {'copy' if write else 'read'}")
    else:
        a = torch.empty(n, device="cuda")
        b = torch.empty(n, device="cuda")
        out = torch.empty(n, device="cuda")
        gn.synth_normal(a, SEED, 1)
        gn.synth_normal(b, SEED, 4)
        passes = gn.STREAM_KINDS[pattern][1]
        kname = f"k_stream<{gn.STREAM_KINDS[pattern][0]}>"
        launch = lambda: gn.synth_stream(pattern, a, b, out)
        what = f"streaming ceiling: {pattern} over 1 GiB buffers ({passes} tensor passes)"
    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record()
        launch()
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    med = ms[len(ms) // 2]
    nbytes = passes * n * 4
    value = nbytes / (med * 1e-3) / 1e9
    print(json.dumps({
        "metric": f"{args.config} achieved HBM GB/s (streaming ceiling, 1 GiB buffers)",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(med, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic N(0,1)",
        "config": {"workload": what},
        "frac_of_peak": round(value / PEAK_GBS, 4), "wall_s_timed": round(wall, 4),
        "best_ms": round(ms[0], 4),
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(value, 1),
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": round(value / PEAK_GBS, 4),
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_ms": round(med, 5),
                     "traffic": None},
        "cpu_baseline": None}), flush=True)


def _host_cpu():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline():
    """fp32 statement of the reference CPU path (oracle/soar_oracle.c, the
    unfused loops of src/nn/layers.cpp), on one core: this thread pinned to
    one CPU (the lowest it may use), one warm-up then the median of 3 runs
    (the reference's idiom, src/main.cpp:675-682).  Config 3 is sampled as
    4 of its 16 groups (the same per-group size, 1/4 of the tensor) to keep
    the run within seconds; config 1 runs at full size (forward only, its
    workload); configs 2 (forward) and 5 (forward + backward, its stress
    input) run one full-size group each (groups are independent, so a
    group's time scales to the config by its group count)."""
    import numpy as np
    import soar_oracle as orc
    eps = float(np.float32(1e-5))
    allowed = os.sched_getaffinity(0)
    core = min(allowed)
    os.sched_setaffinity(0, {core})
    try:
        def run(N, C, HW, G, seed, stress=False, backward=True):
            n = N * C * HW
            x = orc.fill_stress(n, seed) if stress else orc.fill_normal(n, seed, 1)
            gamma = orc.fill_uniform(C, seed, 2, 0.5, 1.5)
            beta = orc.fill_normal(C, seed, 3, 0.0, 0.1)
            dy = orc.fill_normal(n, seed, 4, 0.0, 1e-2) if backward else None
            orc.ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, eps)  # warm-up
            runs = [orc.ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, eps)
                    for _ in range(3)]
            med = lambda k: sorted(r[k] for r in runs)[1]
            return n, med("fwd_s"), med("bwd_s"), sorted(r["fwd_s"] + r["bwd_s"] for r in runs)[1]

        n3, f3, b3, t3 = run(1, 16, 2048 * 2048, 4, SEED + 3)
        n1, f1, _, _ = run(1, 32, 256 * 256, 8, SEED + 1, backward=False)
        n2, f2, _, _ = run(1, 4, 2048 * 2048, 1, SEED + 2, backward=False)
        n5, f5, b5, t5 = run(1, 4, 2048 * 2048, 1, SEED + 5, stress=True)
    finally:
        os.sched_setaffinity(0, allowed)
    group = "one full-size group (N=1 C=4 H=W=2048 G=1), same method"
    return {"value": round(8 * n3 * 4 / t3 / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"config 3 as N=1 C=16 H=W=2048 G=4 (4 of its 16 groups), fwd+bwd, "
                      f"1 warm-up + median of 3 on CPU {core} ({_host_cpu()}, {len(allowed)} "
                      f"CPUs allowed): fwd {f3 * 1e3:.1f} ms, bwd {b3 * 1e3:.1f} ms",
            "config1_fwd": {"ms": round(f1 * 1e3, 3), "GBps": round(3 * n1 * 4 / f1 / 1e9, 3),
                            "shape": "N=1 C=32 H=W=256 G=8, full size, same method"},
            "config2_fwd": {"group_ms": round(f2 * 1e3, 2), "config_ms": round(8 * f2 * 1e3, 1),
                            "GBps": round(3 * n2 * 4 / f2 / 1e9, 3), "shape": group + ", x 8 groups"},
            "config5": {"group_fwd_ms": round(f5 * 1e3, 2), "group_bwd_ms": round(b5 * 1e3, 2),
                        "config_ms": round(4 * t5 * 1e3, 1),
                        "GBps": round(8 * n5 * 4 / t5 / 1e9, 3),
                        "shape": "one full-size group of the stress input (N=1 C=4 H=W=2048 "
                                 "G=1), same method, x 4 groups"},
            "config3_fwd_ms": round(f3 * 1e3, 2), "config3_bwd_ms": round(b3 * 1e3, 2)}


def train_cpu_baseline(H, W, variant):
    """The float64 CPU restatement of one training step (oracle/
    soar_model_ref.py on torch's CPU kernels), best of 2 after a warm-up."""
    import numpy as np
    import torch
    import soar_model_ref as smr
    spec = smr.model_spec(1, 1, {"nano": 0}[variant])
    w = smr.random_weights(spec, SEED)
    img = np.random.default_rng(SEED).normal(0.5, 0.25, size=(1, H, W)).astype(np.float32)
    mask = (np.random.default_rng(SEED + 1).uniform(size=(1, H, W)) < 0.3).astype(np.float32)
    smr.forward_backward(w, img, mask)
    ts = []
    for _ in range(2):
        t0 = time.perf_counter()
        smr.forward_backward(w, img, mask)
        ts.append(time.perf_counter() - t0)
    t = min(ts)
    return {"value": round(1.0 / t, 3), "unit": "images/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"forward+loss+backward of one {H}x{W} image in float64 on the CPU "
                      f"(the oracle's restatement; no optimizer step), best of 2 after 1 "
                      f"warm-up, {t * 1e3:.1f} ms"}


def bench_train(args):
    """Images/s of soar_train_step on one GPU (inputs are host arrays, as
    the C-ABI takes them: the timed step includes their copy to the
    device and the loss read-back, as in the reference's train_step).
    `value` is the default handle, whose steps replay a HIP graph from the
    second step on; `eager_ms_per_step` times a second handle with graphs
    off, which also serves the per-kernel timing pass (a replayed graph
    has no host calls to time)."""
    import numpy as np
    import torch
    import soar_gn as gn
    import soar_model as sm
    variant, H, W = TRAIN_CONFIGS[args.config]
    r = np.random.default_rng(SEED)
    img = r.normal(0.5, 0.25, size=(1, H, W)).astype(np.float32)
    yy, xx = np.mgrid[0:H, 0:W]
    mask = (((yy - H / 2) ** 2 + (xx - W / 3) ** 2) < (min(H, W) / 3) ** 2).astype(np.float32)
    mask = mask[None]

    def timed(m):
        for _ in range(args.warmup):
            m.train_step(img, mask, 1e-3)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            m.train_step(img, mask, 1e-3)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / args.steps

    m = sm.SOAR(1, 1, variant, seed=SEED)
    dt = timed(m)
    graphed = m.graph_info()
    mem = m.memory_info()
    m.close()
    kernels = []
    dt_eager = None
    if not args.no_eager:
        me = sm.SOAR(1, 1, variant, seed=SEED)
        me.set_graph_mode(False)
        dt_eager = timed(me)
    if not args.no_eager and not args.no_kernel_timing:
        gn.prof_summary()  # drop anything recorded so far
        gn.prof_enable(True)
        for _ in range(args.steps):
            me.train_step(img, mask, 1e-3)
        torch.cuda.synchronize()
        gn.prof_enable(False)
        recs = gn.prof_summary()
        total = sum(k["total_ms"] for k in recs) / args.steps
        kernels = [{"kernel": k["kernel"], "ms_per_step": round(k["total_ms"] / args.steps, 4),
                    "launches_per_step": k["launches"] // args.steps}
                   for k in sorted(recs, key=lambda k: -k["total_ms"])[:10]]
        kernels.append({"kernel": "(all timed kernels)", "ms_per_step": round(total, 4)})
    if not args.no_eager:
        me.close()
    out = {
        "metric": f"SOAR {variant} train_step images/s, 1x{H}x{W} fp32",
        "value": round(1.0 / dt, 3), "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.config, "variant": variant, "image": [1, H, W],
                   "loss": "CompositeLoss(0.5, 0.5)", "optimizer": "AdamW lr 1e-3, clip 2.0",
                   "hip_graph": {"on": graphed[0], "graphs": graphed[1]}},
        "eager_ms_per_step": None if dt_eager is None else round(dt_eager * 1e3, 4),
        "roofline": None,
        "kernels_top": kernels,
        "memory": mem,
    }
    if not args.no_cpu_baseline and H * W <= 512 * 512:
        out["cpu_baseline"] = train_cpu_baseline(H, W, variant)
    print(json.dumps(out))


def bench_predict(args):
    """Images/s of soar_predict on one GPU (host image in; probabilities,
    mask and RLE string out, as the reference's C-ABI returns them)."""
    import numpy as np
    import torch
    import soar_model as sm
    variant, H, W = PREDICT_CONFIGS[args.config]
    r = np.random.default_rng(SEED)
    img = r.normal(0.5, 0.25, size=(1, H, W)).astype(np.float32)
    m = sm.SOAR(1, 1, variant, seed=SEED)
    for _ in range(args.warmup):
        m.predict(img)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.predict(img)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    mem = m.memory_info()
    m.close()
    print(json.dumps({
        "metric": f"SOAR {variant} predict images/s, 1x{H}x{W} fp32",
        "value": round(1.0 / dt, 3), "unit": "images/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.config, "variant": variant, "image": [1, H, W],
                   "threshold": 0.5},
        "roofline": None, "memory": mem}))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has "
              "no multi-GPU path.", file=sys.stderr)
        sys.exit(2)
    # torch first: its HIP runtime is the one the process uses, as in the
    # tests (loading libsoar_gn.so first would bind /opt/rocm's instead)
    import torch  # noqa: F401
    tuning = apply_tuning(args)
    if args.config in TRAIN_CONFIGS or args.config in STREAM_CONFIGS or \
            args.config in PREDICT_CONFIGS:
        import torch
        assert torch.cuda.is_available(), "bench.py needs a GPU"
        torch.cuda.set_device(0)
        if args.config in TRAIN_CONFIGS:
            bench_train(args)
        elif args.config in PREDICT_CONFIGS:
            bench_predict(args)
        elif args.config == "stream_sweep":
            bench_stream_sweep(args)
        else:
            bench_stream(args)
        return
    import torch
    import soar_gn as gn

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    gn.lib()
    torch.cuda.set_device(0)

    if args.copy_calibration:
        n = 1 << 28
        a = torch.empty(n, device="cuda")
        b = torch.empty(n, device="cuda")
        gn.synth_normal(a, 1, 1)
        for _ in range(5):
            gn.synth_copy(a, b)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4}))
        return

    if args.config in DW_CONFIGS:
        step = DwStep(gn, args.config, SEED + 7)
    elif args.config in CBA_DW_CONFIGS:
        step = CBADwStep(gn, args.config, SEED + 8)
    elif args.config in ("cba_pw", "cba_pw_unfused"):
        N, C, HW, G, passes, residual, blocks = CONFIGS[args.config]
        step = CBAStep(gn, N, C, HW, G, SEED_OF[args.config], fused=args.config == "cba_pw")
    else:
        N, C, HW, G, passes, residual, blocks = CONFIGS[args.config]
        step = Step(gn, N, C, HW, G, passes, residual, blocks, SEED_OF[args.config])
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    def timed(instrument):
        """K steps between a synchronize and hipEvents on torch's current
        stream (the stream every launch goes to).  With `instrument`, the
        library also brackets each kernel with its own hipEvents."""
        if instrument:
            gn.prof_summary()  # drop anything recorded so far
            gn.prof_enable(True)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            step()
        stop.record()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t0
        recs = []
        if instrument:
            gn.prof_enable(False)
            recs = gn.prof_summary()
        return start.elapsed_time(stop) / args.steps, wall_s, recs

    # `value` comes from the plain timed region; per-kernel events cost a few
    # percent of step time, so the roofline's kernel averages come from an
    # identical instrumented repeat of it.
    ms, wall, _ = timed(False)
    kernels = [] if args.no_kernel_timing else timed(True)[2]
    alg = step.algorithmic_bytes()
    value = alg / (ms * 1e-3) / 1e9

    roofline = None
    kinfo = {}
    blocks = len(step.params)
    for k in kernels:
        avg = k["total_ms"] / k["launches"]
        per_step = k["launches"] / args.steps
        # bytes of one launch: the kernel's passes over the tensor, split
        # evenly over its launches (equal-sized unit batches)
        if hasattr(step, "kernel_bytes"):
            per_launch = step.kernel_bytes(k["kernel"])
        else:
            per_launch = PASSES.get(k["kernel"], 0) * step.T * blocks / per_step
        kinfo[k["kernel"]] = {"launches_per_step": per_step, "avg_launch_ms": round(avg, 5),
                              "bytes_per_launch": int(per_launch),
                              "GBps": round(per_launch / (avg * 1e-3) / 1e9, 1)
                              if per_launch else None}
        flops = step.kernel_flops(k["kernel"]) if hasattr(step, "kernel_flops") else 0
        if flops:
            tf = flops / (avg * 1e-3) / 1e12
            kinfo[k["kernel"]]["TFLOPs"] = round(tf, 2)
            if isinstance(step, (DwStep, CBADwStep)):  # vector FMAs, not the matrix cores
                kinfo[k["kernel"]]["valu_frac"] = round(tf / PEAK_VALU_F32, 4)
            else:
                kinfo[k["kernel"]]["mfma_frac"] = round(tf / PEAK_MFMA_F32, 4)
    if kernels:
        dom = max(kernels, key=lambda k: k["total_ms"])
        kd = kinfo[dom["kernel"]]
        achieved = kd["GBps"]
        tr = traffic_from_profiles(args.config)
        roofline = {"bound": "hbm", "kernel": dom["kernel"], "achieved": achieved,
                    "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4),
                    "algorithmic_bytes_per_launch": kd["bytes_per_launch"],
                    "avg_launch_ms": kd["avg_launch_ms"],
                    "traffic": tr.get(dom["kernel"]) if tr else None}
        if "mfma_frac" in kd:
            # the conv is near the ridge: also its place under the fp32
            # matrix-core roof
            roofline["mfma"] = {"achieved": kd["TFLOPs"], "peak": PEAK_MFMA_F32,
                                "unit": "TFLOP/s", "frac": kd["mfma_frac"]}
        if "valu_frac" in kd:
            roofline["valu"] = {"achieved": kd["TFLOPs"], "peak": PEAK_VALU_F32,
                                "unit": "TFLOP/s", "frac": kd["valu_frac"]}

    cpu = None
    if not args.no_cpu_baseline and args.config == "cfg3":
        cpu = cpu_baseline()

    if isinstance(step, DwStep):
        data = (f"synthetic: x~N(0,1), w~U(-1/K,1/K), b~N(0,0.1), dy~N(0,1e-2); "
                f"splitmix64/Box-Muller seed {SEED + 7}")
        cfg = {**step.config(), "algorithmic_bytes_per_step": alg}
    elif isinstance(step, CBADwStep):
        data = (f"synthetic: x~N(0,1), w~U(-1/K,1/K), gamma~U(0.5,1.5), beta~N(0,0.1), "
                f"dy~N(0,1e-2); splitmix64/Box-Muller seed {SEED + 8}")
        cfg = {**step.config(), "algorithmic_bytes_per_step": alg}
    else:
        data = (f"synthetic: x~N(0,1), gamma~U(0.5,1.5), beta~N(0,0.1), dy~N(0,1e-2); "
                f"splitmix64/Box-Muller seed {SEED_OF[args.config]}")
        cfg = {"workload": {"cfg3": "GroupNorm+SiLU fwd+bwd, BASELINE config 3",
                            "cfg1_fwd": "GroupNorm+SiLU fwd, BASELINE config 1 (8 MiB: "
                                        "cache-resident, not a roofline config)",
                            "cfg2_fwd": "GroupNorm+SiLU fwd, BASELINE config 2",
                            "cfg4_chain": "6 x (x + SiLU(GN(x))) fwd+bwd, BASELINE config 4",
                            "cfg5": "GroupNorm+SiLU fwd+bwd shape of BASELINE config 5",
                            "cba_pw": "CBA fwd+bwd: pointwise conv 64->64 + GN + SiLU, GN "
                                      "stats in the conv epilogue, fused backward (dz in "
                                      "registers), config 3 GroupNorm shape",
                            "cba_pw_unfused": "CBA fwd+bwd: pointwise conv 64->64 + GN + SiLU, "
                                              "GN stats in the conv epilogue, backward as GN "
                                              "backward then conv backward, config 3 GroupNorm "
                                              "shape"}
               [args.config],
               "N": N, "C": C, "H": int(HW ** 0.5), "W": int(HW ** 0.5), "G": G,
               "eps": 1e-5, "blocks": blocks, "residual": residual,
               **({"C_in": CBA_C_IN} if args.config.startswith("cba_pw") else {}),
               "algorithmic_bytes_per_step": alg}
    if tuning:
        cfg["tuning"] = tuning
    out = {
        "metric": METRIC if args.config == "cfg3" else f"{args.config} achieved HBM GB/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": data,
        "config": cfg,
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "wall_s_timed": round(wall, 4),
        "roofline": roofline,
        "kernels": kinfo,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
