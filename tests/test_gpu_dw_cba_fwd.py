"""Parity of the fused depthwise CBA forward (soar_dw_conv_gn_silu_forward)
through the C-ABI of libsoar_gn.so.

The depthwise convolution's epilogue computes the GroupNorm statistics of
its own outputs (each block's tile column as float64 (mean, M2) partials),
the finish combines them with the tiles' element counts, and the apply
follows, so no statistics pass re-reads z.  Each case checks:
  z:           bit for bit soar_dw_conv_forward's output (the same kernel
               arithmetic; the epilogue only adds the sums);
  mean, rstd:  against the float64 oracle on the device's own z at the
               statistics bar |d mean| <= 1e-5 max(|mean|, std),
               |d rstd| / rstd <= 1e-5;
  y:           against the float64 oracle at |d| <= 1e-4 (1 + |truth|);
  the path:    the kernel timers show the epilogue kernel and no statistics
               pass for shapes with a tiled kernel and units above the
               one-launch size, and the stand-alone path otherwise;
and two calls agree bit for bit.
"""
import numpy as np
import pytest

from test_gpu_parity import EPS, assert_stats, assert_vals, dev, host

pytestmark = pytest.mark.gpu


def _inputs(seed, N, C, H, W, K, kind):
    r = np.random.default_rng(seed)
    if kind == "offset":
        x = (1e3 + 1e-2 * r.standard_normal((N, C, H, W))).astype(np.float32)
    else:
        x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = (r.uniform(-1.0, 1.0, (C, K, K)) / K).astype(np.float32)
    b = (0.1 * r.standard_normal(C)).astype(np.float32)
    gm = r.uniform(0.5, 1.5, C).astype(np.float32)
    bt = (0.1 * r.standard_normal(C)).astype(np.float32)
    return x, w, b, gm, bt


CASES = [
    # (N, C, H, W, K, S, D, G, silu, kind, bias, fused)
    (1, 16, 256, 256, 3, 1, 1, 4, True, "normal", False, True),   # k3, two rows per thread
    (2, 8, 300, 200, 3, 1, 1, 2, True, "normal", True, True),     # ragged tiles, two samples, bias
    (1, 16, 200, 130, 5, 1, 1, 4, False, "normal", False, True),  # k5 (LKR), no SiLU
    (1, 8, 257, 190, 7, 1, 1, 2, True, "normal", False, True),    # k7 (LKR), ragged both ways
    (1, 16, 256, 256, 3, 2, 1, 4, True, "normal", True, True),    # Down.dw: k3 stride 2
    (1, 8, 200, 200, 3, 1, 3, 2, True, "normal", False, True),    # Ctx dilation 3
    (1, 8, 160, 170, 3, 1, 5, 2, True, "normal", False, True),    # Ctx dilation 5
    (1, 8, 128, 128, 3, 1, 2, 2, True, "normal", False, True),    # dilation 2
    (1, 8, 256, 256, 7, 1, 1, 4, True, "offset", False, True),    # |mean| >> std: the shifts
    (3, 4, 130, 66, 5, 1, 1, 1, True, "normal", True, True),      # three samples, one group
    (1, 8, 32, 32, 3, 1, 1, 2, True, "normal", False, False),     # small units: one-launch GN
    (1, 8, 128, 128, 9, 1, 1, 2, True, "normal", False, False),   # K = 9: no tiled kernel
]


def _launches():
    import soar_gn
    return {r["kernel"]: r["launches"] for r in soar_gn.prof_summary()}


@pytest.mark.parametrize("N,C,H,W,K,S,D,G,silu,kind,bias,fused", CASES)
def test_dw_conv_gn_forward_matches_oracle(gpu, oracle, N, C, H, W, K, S, D, G, silu, kind,
                                           bias, fused):
    print(f"dw_conv_gn_forward N={N} C={C} {H}x{W} K={K} S={S} D={D} G={G} silu={silu} "
          f"{kind} bias={bias}", flush=True)
    x, w, b, gm, bt = _inputs(N * 7 + C + H + W + K, N, C, H, W, K, kind)
    pad = D * (K - 1) // 2
    xd, wd, gd, bd = dev(x), dev(w), dev(gm), dev(bt)
    bias_d = dev(b) if bias else None
    z_ref = gpu.dw_conv_forward(xd, wd, bias_d, pad, S, D)
    gpu.prof_summary()  # drop earlier records
    gpu.prof_enable(True)
    try:
        z, y, st = gpu.dw_conv_gn_silu_forward(xd, wd, bias_d, gd, bd, G, pad, S, D, eps=EPS,
                                               silu=silu)
        import torch
        torch.cuda.synchronize()
        runs = _launches()
    finally:
        gpu.prof_enable(False)
    assert ("dw_conv_stats" in runs) == fused, runs
    assert ("gn_stats_partial" in runs) == (not fused and "gn_small_fwd" not in runs), runs
    assert np.array_equal(host(z), host(z_ref)), "z differs from soar_dw_conv_forward"
    Ho, Wo = z.shape[2], z.shape[3]
    HW = Ho * Wo
    zh = host(z).reshape(-1)
    yt, mt, rt = oracle.gn_silu_fwd_f64(zh, gm, bt, N, C, HW, G, EPS, silu=silu)
    assert_stats(host(st.mean), host(st.rstd), mt, rt, "stats")
    assert_vals(host(y), yt, "y")
    # the saved mean residual: mean + mean_lo is the float64 mean to its rounding
    eff = host(st.mean).astype(np.float64) + host(st.mean_lo).astype(np.float64)
    std_t = np.sqrt(np.maximum(1.0 / rt ** 2 - EPS, 0.0))
    assert np.max(np.abs(eff - mt) / np.maximum(np.abs(mt), std_t)) <= 1e-6
    # two calls agree bit for bit
    z2, y2, st2 = gpu.dw_conv_gn_silu_forward(xd, wd, bias_d, gd, bd, G, pad, S, D, eps=EPS,
                                              silu=silu)
    assert np.array_equal(host(y), host(y2)) and np.array_equal(host(st.rstd), host(st2.rstd))


FOLD_CASES = [
    # (N, C, H, W, K, S, D, G): tile groups per unit (cpg * tpp) from a few
    # dozen to several hundred
    (1, 16, 512, 512, 3, 1, 1, 8),    # SOAR Nano gate_dw at 1024^2: 512 partials
    (1, 32, 256, 256, 7, 1, 1, 8),    # LKR k7: 256
    (2, 64, 100, 130, 5, 1, 1, 8),    # ragged tiles, two samples
    (1, 16, 256, 256, 3, 2, 1, 4),    # stride 2
]


@pytest.mark.parametrize("N,C,H,W,K,S,D,G", FOLD_CASES)
def test_dw_conv_gn_forward_folded_finish(gpu, oracle, N, C, H, W, K, S, D, G):
    """The finish of the tile-group partials folded into the apply
    (SOAR_TUNE_FOLD_MAX at or above the unit's partials): no finish launch,
    and mean, rstd, mean_lo and y bit for bit those of the separate finish
    (0: always separate), which the oracle checks."""
    import torch
    print(f"dw_conv_gn_forward folded N={N} C={C} {H}x{W} K={K} S={S} D={D} G={G}", flush=True)
    x, w, b, gm, bt = _inputs(N + C + H + K + 11, N, C, H, W, K, "normal")
    pad = D * (K - 1) // 2
    xd, wd, gd, bd = dev(x), dev(w), dev(gm), dev(bt)
    old = gpu.tune_get(gpu.TUNE_FOLD_MAX)
    runs = {}
    try:
        for fold in (0, 4096):
            gpu.tune(gpu.TUNE_FOLD_MAX, fold)
            gpu.prof_summary()
            gpu.prof_enable(True)
            try:
                z, y, st = gpu.dw_conv_gn_silu_forward(xd, wd, dev(b), gd, bd, G, pad, S, D,
                                                       eps=EPS)
                torch.cuda.synchronize()
                names = _launches()
            finally:
                gpu.prof_enable(False)
            assert "dw_conv_stats" in names, names
            assert ("gn_stats_finish" in names) == (fold == 0), names
            runs[fold] = [host(t) for t in (z, y, st.mean, st.rstd, st.mean_lo)]
    finally:
        gpu.tune(gpu.TUNE_FOLD_MAX, old)
    for a, c in zip(runs[0], runs[4096]):
        assert np.array_equal(a, c)
    z, y, mean, rstd = runs[4096][:4]
    Ho, Wo = z.shape[2], z.shape[3]
    yt, mt, rt = oracle.gn_silu_fwd_f64(z.reshape(-1), gm, bt, N, C, Ho * Wo, G, EPS)
    assert_stats(mean, rstd, mt, rt, "folded stats")
    assert_vals(y, yt, "folded y")


def test_dw_conv_gn_forward_full_size_k7(gpu, oracle):
    """The CBA LKR block's k7 depthwise conv at BASELINE config 3's shape
    (1 x 64 x 2048^2, G = 16): whole-tensor statistics against the float64
    oracle on the device z, y at sampled indices against the closed form on
    oracle statistics, z bit for bit the stand-alone convolution's."""
    import torch
    N, C, H, W, K, G = 1, 64, 2048, 2048, 7, 16
    print("dw_conv_gn_forward full size 1x64x2048^2 k7 G=16", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261207)
    xd = torch.randn((N, C, H, W), generator=gen, device="cuda")
    wd = (torch.rand((C, K, K), generator=gen, device="cuda") * 2 - 1) / K
    gd = torch.rand(C, generator=gen, device="cuda") + 0.5
    bd = 0.1 * torch.randn(C, generator=gen, device="cuda")
    z, y, st = gpu.dw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, 3, eps=EPS)
    z_ref = gpu.dw_conv_forward(xd, wd, None, 3)
    torch.cuda.synchronize()
    assert torch.equal(z, z_ref)
    del z_ref
    zh = host(z).reshape(-1)
    gh, bh = host(gd), host(bd)
    HW = H * W
    _, mt, rt = oracle.gn_silu_fwd_f64(zh, gh, bh, N, C, HW, G, EPS, want_y=False)
    assert_stats(host(st.mean), host(st.rstd), mt, rt, "full-size stats")
    rng = np.random.default_rng(7)
    idx = rng.integers(0, N * C * HW, 200000)
    c = idx // HW
    u = c // (C // G)
    zz = gh[c] * ((zh[idx].astype(np.float64) - mt[u]) * rt[u]) + bh[c]
    assert_vals(host(y).reshape(-1)[idx], zz / (1 + np.exp(-zz)), "sampled y")


def test_dw_conv_gn_forward_errors(gpu):
    import torch
    g = gpu
    N, C, H, W, K, G = 1, 8, 128, 128, 3, 2
    t = lambda *s: torch.zeros(s, dtype=torch.float32, device="cuda")
    need = g.dw_conv_gn_workspace_bytes(N, C, H, W, H, W, K, 1, 1, 1, G)
    gn_only = g.workspace_bytes(N, C, H * W, G)
    assert need > gn_only  # the tile-group partials after the GroupNorm workspace
    small = torch.empty(need - 256, dtype=torch.uint8, device="cuda")
    with pytest.raises(g.SoarError):
        g.dw_conv_gn_silu_forward(t(N, C, H, W), t(C, K, K), None, None, None, G, 1, ws=small)
    assert "workspace" in g.last_error()
    with pytest.raises(g.SoarError):
        g.dw_conv_gn_silu_forward(t(N, C, H, W), t(C, K, K), None, None, None, 3, 1)  # C % G
