"""The HIP path next to the reference's own fp32 formulas at every BASELINE
config.

ref_gn_silu_fwd_bwd_f32 (oracle/soar_oracle.c) restates the reference's CPU
GroupNorm -> SiLU [-> add] forward and backward in fp32 as compiled
(src/nn/layers.cpp:694-707 statistics, :712-721 apply, :760-769 / :789-795
SiLU, :545-617 GroupNorm backward).  For each config the test runs that
restatement, the HIP kernels through the C-ABI and the float64 oracle on
the same seeded inputs, and reports three deltas per output, each the
largest |a - b| / (1 + |truth|) (statistics: |d mean| / max(|mean|, std)
and |d rstd| / rstd):
  hip_truth  the build against float64 truth (the parity bar: 1e-4, 1e-5)
  ref_truth  the reference's own fp32 result against float64 truth
  hip_ref    the build against the reference's fp32 result
and asserts hip_truth within the bar and |hip - ref| <= |ref - truth| + bar
elementwise.  Groups are independent, so configs 2, 3 and 5 run one
full-size group (the first 4 planes of the config's seeded tensors, whose
generator is counter-based: the group's values are the tensor's first
elements); config 1 runs whole and config 4 runs its first block on one
sample.  Each case prints one line "REF_F32 {json}" with the deltas.
"""
import json

import numpy as np
import pytest

from test_gpu_parity import EPS, STAT_TOL, VAL_TOL, dev, host

pytestmark = pytest.mark.gpu

CONFIGS = {
    # name: (N, C, HW, G, kind, backward, residual, what)
    "config1": (1, 32, 256 * 256, 8, "normal", True, False, "whole tensor"),
    "config2": (1, 4, 2048 * 2048, 1, "normal", False, False, "one group of 1x32x2048^2 G=8"),
    "config3": (1, 4, 2048 * 2048, 1, "normal", True, False, "one group of 1x64x2048^2 G=16"),
    "config4": (1, 128, 1024 * 1024, 32, "normal", True, True,
                "block 0 of the chain, sample 0 of 2x128x1024^2 G=32"),
    "config5": (1, 4, 2048 * 2048, 1, "stress", True, False, "one group of 1x16x2048^2 G=4"),
}


def _scaled(a, b, truth):
    return np.abs(np.asarray(a, np.float64) - b) / (1.0 + np.abs(truth))


@pytest.mark.parametrize("name", list(CONFIGS))
def test_hip_against_reference_fp32(gpu, oracle, name):
    N, C, HW, G, kind, backward, residual, what = CONFIGS[name]
    seed = 20261201 + int(name[-1])
    print(f"ref fp32 {name}: N={N} C={C} HW={HW} G={G} {kind} ({what})", flush=True)
    n = N * C * HW
    x = oracle.fill_stress(n, seed) if kind == "stress" else oracle.fill_normal(n, seed, 1)
    gamma = oracle.fill_uniform(C, seed, 2, 0.5, 1.5)
    beta = oracle.fill_normal(C, seed, 3, 0.0, 0.1)
    dy = oracle.fill_normal(n, seed, 4, 0.0, 1e-2) if backward else None

    # the reference's fp32 formulas, float64 truth, and the build
    ref = oracle.ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, EPS,
                                         residual=residual)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, True, residual)
    xd = dev(x).view(N, C, HW)
    y, st = gpu.gn_silu_forward(xd, dev(gamma), dev(beta), G, eps=EPS, residual=residual)
    out = {"config": name, "shape": [N, C, HW, G], "what": what}
    std_t = np.sqrt(np.maximum(1.0 / rt ** 2 - EPS, 0.0))
    mscale = np.maximum(np.abs(mt), std_t)
    for key, got_ref, got_hip, truth, bar in (
            ("mean", ref["mean"], host(st.mean), mt, STAT_TOL),
            ("rstd", ref["rstd"], host(st.rstd), rt, STAT_TOL)):
        sc = mscale if key == "mean" else rt
        d_hip = np.abs(np.asarray(got_hip, np.float64) - truth) / sc
        d_ref = np.abs(np.asarray(got_ref, np.float64) - truth) / sc
        d_hr = np.abs(np.asarray(got_hip, np.float64) - got_ref) / sc
        out[key] = {"hip_truth": float(d_hip.max()), "ref_truth": float(d_ref.max()),
                    "hip_ref": float(d_hr.max())}
        assert d_hip.max() <= bar, (key, d_hip.max())
        assert np.all(d_hr <= d_ref + bar), key
    pairs = [("y", ref["y"], host(y).reshape(-1), yt)]
    if backward:
        dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G, True,
                                               residual)
        dx, dg, db = gpu.gn_silu_backward(dev(dy).view(N, C, HW), xd, dev(gamma), dev(beta),
                                          st, G, residual=residual)
        pairs += [("dx", ref["dx"], host(dx).reshape(-1), dxt),
                  ("dgamma", ref["dgamma"], host(dg), dgt),
                  ("dbeta", ref["dbeta"], host(db), dbt)]
    for key, got_ref, got_hip, truth in pairs:
        d_hip = _scaled(got_hip, truth, truth)
        d_ref = _scaled(got_ref, truth, truth)
        d_hr = _scaled(got_hip, np.asarray(got_ref, np.float64), truth)
        out[key] = {"hip_truth": float(d_hip.max()), "ref_truth": float(d_ref.max()),
                    "hip_ref": float(d_hr.max())}
        assert d_hip.max() <= VAL_TOL, (key, d_hip.max())
        assert np.all(d_hr <= d_ref + VAL_TOL), key
    out["ref_cpu_s"] = {"fwd": ref["fwd_s"], "bwd": ref["bwd_s"]}
    print("REF_F32 " + json.dumps(out), flush=True)
