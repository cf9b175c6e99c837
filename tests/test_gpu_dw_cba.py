"""Parity of the fused depthwise CBA backward (soar_dw_cba_backward) through
the C-ABI of libsoar_gn.so.

For a stride-1 depthwise convolution with "same" padding the fused kernel
forms dz, the GroupNorm(+SiLU) input gradient, over each tile and its halo
in LDS with the GroupNorm dx pass's arithmetic, and computes the
convolution's dx and weight gradient from it without storing dz.  Each case
checks, on the same device forward:
  dz:      the stand-alone device GroupNorm backward (soar_gn_silu_backward
           on its multi-kernel path, whose reduction and dx arithmetic the
           fused kernel shares) against the float64 oracle at the GroupNorm
           bar |d| <= 1e-4 (1 + |truth|);
  dx, dW:  against the float64 depthwise backward of that device dz at the
           fp32 bound of their sums (test_gpu_dw_conv's bars), so a wrong dz
           inside the fused kernel (a coefficient, a halo element, an edge)
           fails;
  dgamma, dbeta: bit for bit equal to the stand-alone GroupNorm backward;
and the fused result against the unfused entry-point path (TUNE_DW_CBA_MIN
= 0): the same FMA order, so dx agrees bit for bit, and so does dW on these
grids, where both weight gradients take one tile per block (on larger grids
the fused kernel groups 2 or 8 tiles per block where the stand-alone one
groups 4 or 8, so dW may differ in its last bits).
"""
import numpy as np
import pytest

from test_gpu_parity import EPS, dev, host

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


@pytest.fixture
def fused(gpu):
    """The fused kernel for every size, and the stand-alone GroupNorm
    backward on its multi-kernel path (no one-launch small-unit kernel, no
    folded finish)."""
    keys = (gpu.TUNE_DW_CBA_MIN, gpu.TUNE_SMALL_UNIT, gpu.TUNE_FOLD_MAX)
    old = {k: gpu.tune_get(k) for k in keys}
    gpu.tune(gpu.TUNE_DW_CBA_MIN, 1)
    gpu.tune(gpu.TUNE_SMALL_UNIT, 0)
    gpu.tune(gpu.TUNE_FOLD_MAX, 0)
    yield gpu
    for k, v in old.items():
        gpu.tune(k, v)


def _inputs(seed, N, C, H, W, K, kind="normal"):
    r = np.random.default_rng(seed)
    if kind == "offset":
        x = (1e3 + 1e-2 * r.standard_normal((N, C, H, W))).astype(np.float32)
    else:
        x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = (r.uniform(-1.0, 1.0, (C, K, K)) / K).astype(np.float32)
    gm = r.uniform(0.5, 1.5, C).astype(np.float32)
    bt = (0.1 * r.standard_normal(C)).astype(np.float32)
    dy = (1e-2 * r.standard_normal((N, C, H, W))).astype(np.float32)
    return x, w, gm, bt, dy


def _within(got, truth, bound, name):
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - np.asarray(truth).reshape(-1))
    b = np.asarray(bound).reshape(-1)
    ratio = err / (b + 1e-30)
    i = int(np.argmax(ratio))
    assert ratio[i] <= 1.0, f"{name}: err {err[i]:.3e} > bound {b[i]:.3e} at {i}"


def _dw_bounds(dz, x, w, pad, D, oracle):
    """fp32 bounds of the depthwise dx (K*K-term sums) and dW (N*H*W-term
    sums): the float64 backward of |dz|, |x|, |w|."""
    N, C, H, W = x.shape
    K = w.shape[-1]
    ax, aw, ad = np.abs(x), np.abs(w), np.abs(dz)
    mx, mw, _ = oracle.dw_bwd_f64(ad, ax, aw, N, C, H, W, K, pad, 1, D)
    return (K * K + 2) * U32 * mx, (N * H * W + 2) * U32 * mw


CASES = [
    # (N, C, H, W, K, D, G, silu, kind)
    (1, 16, 64, 64, 3, 1, 4, True, "normal"),      # k3, exact tiles
    (2, 8, 100, 130, 3, 1, 2, True, "normal"),     # ragged tiles, two samples
    (1, 32, 48, 72, 5, 1, 8, False, "normal"),     # k5 (LKR), no SiLU
    (1, 8, 33, 70, 7, 1, 2, True, "normal"),       # k7 (LKR): halo wider than the tail
    (1, 16, 96, 96, 3, 3, 4, True, "normal"),      # Ctx dilation 3
    (1, 8, 70, 40, 3, 5, 2, True, "normal"),       # Ctx dilation 5, halo > tile edge
    (1, 8, 64, 64, 3, 2, 2, True, "normal"),       # dilation 2
    (3, 4, 17, 9, 7, 1, 1, True, "normal"),        # planes smaller than the halo
    (1, 8, 64, 64, 7, 1, 4, True, "offset"),       # large mean offset: the mean residual
    (1, 8, 64, 64, 3, 1, 4, False, "offset"),
]


def _check_case(g, oracle, seed, N, C, H, W, K, D, G, silu, kind):
    pad = (K - 1) * D // 2
    print(f"dw_cba_backward N={N} C={C} {H}x{W} K={K} D={D} G={G} silu={silu} {kind}",
          flush=True)
    x, w, gm, bt, dy = _inputs(seed, N, C, H, W, K, kind)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z = g.dw_conv_forward(xd, wd, None, pad, 1, D)
    _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS, silu=silu)
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G, silu=silu)
    dx, dw, dg, db = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, silu=silu)
    HW = H * W
    zh, dzh = host(z).astype(np.float32), host(dz).astype(np.float32)

    _, m64, r64 = oracle.gn_silu_fwd_f64(zh, gm, bt, N, C, HW, G, EPS, silu=silu, want_y=False)
    tdz, tdg, tdb = oracle.gn_silu_bwd_f64(dy, zh, gm, bt, m64, r64, N, C, HW, G, silu=silu)
    _within(dzh, tdz, 1e-4 * (1.0 + np.abs(tdz)), "dz")
    _within(host(dg), tdg, 1e-4 * (1.0 + np.abs(tdg)), "dgamma")
    _within(host(db), tdb, 1e-4 * (1.0 + np.abs(tdb)), "dbeta")
    assert np.array_equal(host(dg), host(dg_u)) and np.array_equal(host(db), host(db_u))

    tx, tw, _ = oracle.dw_bwd_f64(dzh, x, w, N, C, H, W, K, pad, 1, D)
    bx, bw = _dw_bounds(dzh, x, w, pad, D, oracle)
    _within(host(dx), tx, bx, "dx")
    _within(host(dw), tw, bw, "dW")

    # the unfused entry-point path: the same terms in the same order
    g.tune(g.TUNE_DW_CBA_MIN, 0)
    try:
        ux, uw, ug, ub = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, silu=silu)
    finally:
        g.tune(g.TUNE_DW_CBA_MIN, 1)
    for a, b_, name in ((ux, dx, "dx"), (uw, dw, "dW"), (ug, dg, "dgamma"), (ub, db, "dbeta")):
        assert np.array_equal(host(a), host(b_)), name


@pytest.mark.parametrize("N,C,H,W,K,D,G,silu,kind", CASES)
def test_dw_cba_backward_matches_oracle(fused, oracle, N, C, H, W, K, D, G, silu, kind):
    _check_case(fused, oracle, N * 17 + C * 5 + H + K * 3 + D, N, C, H, W, K, D, G, silu, kind)


@pytest.mark.parametrize("N,C,H,W,K,D,G,silu,kind", [CASES[i] for i in (0, 1, 2, 3, 8)] + [
    (1, 16, 512, 512, 3, 1, 8, True, "normal"),    # SOAR Nano at 1024^2: 64 partials a plane
    (1, 128, 64, 64, 7, 1, 2, True, "normal"),     # 64 planes a unit
])
def test_dw_cba_backward_folded_finish(fused, N, C, H, W, K, D, G, silu, kind):
    """The GroupNorm backward's finish folded into the fused kernel (every
    block forms its unit's plane and unit sums from the reduction's
    partials; SOAR_TUNE_FOLD_MAX 2048): no finish launch, and dx, dW,
    dgamma, dbeta bit for bit those of the separate finish (0)."""
    import torch
    g = fused
    pad = (K - 1) * D // 2
    print(f"dw_cba_backward folded N={N} C={C} {H}x{W} K={K} D={D} G={G}", flush=True)
    x, w, gm, bt, dy = _inputs(N * 13 + C + H + K, N, C, H, W, K, kind)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z = g.dw_conv_forward(xd, wd, None, pad, 1, D)
    _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS, silu=silu)
    runs = {}
    for fold in (0, 2048):
        g.tune(g.TUNE_FOLD_MAX, fold)
        g.prof_summary()
        g.prof_enable(True)
        try:
            out = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, silu=silu)
            torch.cuda.synchronize()
            names = {r["kernel"] for r in g.prof_summary()}
        finally:
            g.prof_enable(False)
        assert "dw_cba_bwd" in names, names
        assert ("gn_bwd_finish" in names) == (fold == 0), names
        runs[fold] = [host(t) for t in out]
    for a, b, name in zip(runs[0], runs[2048], ("dx", "dW", "dgamma", "dbeta")):
        assert np.array_equal(a, b), name


def _sweep_cases(n=20, seed=20261205):
    """Seeded random depthwise CBA blocks: every tiled (K, dilation) with
    "same" padding, 1-3 samples, 1-8 channels per group, planes from a
    single row or column to several ragged tiles, both activations, data
    with a large mean offset; then grids large enough that a block walks
    2 and 4 tiles down its plane (ragged last group)."""
    r = np.random.default_rng(seed)
    kd = [(3, 1), (3, 2), (3, 3), (3, 5), (5, 1), (7, 1)]
    out = []
    for i in range(n):
        K, D = kd[i % len(kd)]
        G = int(r.choice([1, 2, 4, 8]))
        C = G * int(r.integers(1, 9))
        N = int(r.integers(1, 4))
        H = int(r.choice([1, int(r.integers(2, 40)), int(r.integers(40, 140)),
                          int(r.integers(40, 140))]))
        W = int(r.choice([1, int(r.integers(2, 70)), int(r.integers(70, 200)),
                          int(r.integers(70, 200))]))
        silu = bool(r.integers(0, 2))
        kind = "offset" if r.random() < 0.2 else "normal"
        out.append((int(r.integers(1 << 30)), N, C, H, W, K, D, G, silu, kind))
    out.append((11, 2, 64, 300, 260, 3, 1, 16, True, "normal"))   # 2 tiles per block
    out.append((12, 2, 64, 520, 256, 7, 1, 16, True, "normal"))   # 4 tiles per block
    return out


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: "s{}-n{}c{}-{}x{}-k{}d{}".format(
    c[0] % 1000, c[1], c[2], c[3], c[4], c[5], c[6]))
def test_dw_cba_backward_seeded_sweep(fused, oracle, case):
    _check_case(fused, oracle, *case)


@pytest.mark.parametrize("want_dw,accumulate", [(True, True), (False, False), (False, True)])
def test_dw_cba_backward_outputs_and_accumulation(fused, oracle, want_dw, accumulate):
    g = fused
    N, C, H, W, K, D, G = 2, 16, 80, 96, 5, 1, 4
    pad = 2
    x, w, gm, bt, dy = _inputs(91, N, C, H, W, K)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z = g.dw_conv_forward(xd, wd, None, pad, 1, D)
    _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS)
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G)
    r = np.random.default_rng(8)
    dx0 = r.standard_normal((N, C, H, W)).astype(np.float32)
    dw0 = r.standard_normal((C, K, K)).astype(np.float32)
    p0 = r.standard_normal(C).astype(np.float32)
    dwd = dev(dw0)
    dx, dw, dg, db = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D,
                                       dx=dev(dx0) if accumulate else None, dweight=dwd,
                                       dgamma=dev(p0), dbeta=dev(p0), want_dw=want_dw,
                                       accumulate_dx=accumulate)
    dzh = host(dz)
    tx, tw, _ = oracle.dw_bwd_f64(dzh, x, w, N, C, H, W, K, pad, 1, D)
    bx, bw = _dw_bounds(dzh, x, w, pad, D, oracle)
    t = tx.reshape(-1) + (dx0.reshape(-1).astype(np.float64) if accumulate else 0.0)
    _within(host(dx), t, bx.reshape(-1) + 2.0 ** -23 * np.abs(t), "dx")
    if want_dw:
        t = tw.reshape(-1) + dw0.reshape(-1).astype(np.float64)
        _within(host(dw), t, bw.reshape(-1) + 2.0 ** -23 * np.abs(t), "dW")
    else:
        assert dw is None and np.array_equal(host(dwd), dw0)
    for got, u, name in ((dg, dg_u, "dgamma"), (db, db_u, "dbeta")):
        u = host(u).astype(np.float64)
        t = p0.astype(np.float64) + u
        _within(host(got), t, 2.0 ** -24 * (np.abs(u) + np.abs(t)) + 1e-30, name)


@pytest.mark.parametrize("K,D", [(3, 1), (7, 1), (3, 5)])
def test_dw_cba_backward_single_outputs_in_queried_workspace(fused, K, D):
    """dW alone runs the fused kernel without its dx product, dx alone
    without its weight-gradient sums, and dgamma / dbeta alone the GroupNorm
    backward only; each within the workspace the size query returns (the
    fused path's, smaller than dz) and bit for bit the full call's outputs."""
    import torch
    g = fused
    N, C, H, W, G = 2, 16, 70, 100, 4
    pad = (K - 1) * D // 2
    print(f"dw_cba_backward single outputs K={K} D={D}", flush=True)
    x, w, gm, bt, dy = _inputs(57 + K + D, N, C, H, W, K)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z = g.dw_conv_forward(xd, wd, None, pad, 1, D)
    _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS)
    need = g.dw_cba_backward_workspace_bytes(N, C, H, W, H, W, K, pad, 1, D, G)
    assert 0 < need < N * C * H * W * 4
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    fx, fw, fg, fb = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, ws=ws)
    _, ow, _, _ = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, want_dx=False,
                                    want_params=False, ws=ws)
    ox, _, _, _ = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, want_dw=False,
                                    want_params=False, ws=ws)
    _, _, pg, pb = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, pad, 1, D, want_dx=False,
                                     want_dw=False, ws=ws)
    for a, b_, name in ((ox, fx, "dx"), (ow, fw, "dW"), (pg, fg, "dgamma"), (pb, fb, "dbeta")):
        assert np.array_equal(host(a), host(b_)), name


def test_dw_cba_backward_unfused_shapes(gpu, oracle):
    """Shapes outside the fused kernel (stride 2, asymmetric padding, a
    generic K) run the two stand-alone calls through the same entry point."""
    g = gpu
    for (K, pad, S, D) in ((3, 1, 2, 1), (3, 0, 1, 1), (4, 2, 1, 1)):
        N, C, H, W, G = 1, 8, 40, 36, 2
        x, w, gm, bt, _ = _inputs(K + 10 * pad + S, N, C, H, W, K)
        xd, wd, gd, bd = dev(x), dev(w), dev(gm), dev(bt)
        z = g.dw_conv_forward(xd, wd, None, pad, S, D)
        Ho, Wo = z.shape[2], z.shape[3]
        dy = (1e-2 * np.random.default_rng(K).standard_normal((N, C, Ho, Wo))).astype(np.float32)
        _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS)
        dz, dg_u, db_u = g.gn_silu_backward(dev(dy), z, gd, bd, st, G)
        ux, uw, _ = g.dw_conv_backward(dz, xd, wd, pad, S, D, want_db=False)
        dx, dw, dg, db = g.dw_cba_backward(dev(dy), z, xd, wd, gd, bd, st, G, pad, S, D)
        for a, b_, name in ((dx, ux, "dx"), (dw, uw, "dW"), (dg, dg_u, "dgamma"),
                            (db, db_u, "dbeta")):
            assert np.array_equal(host(a), host(b_)), (K, pad, S, name)


def test_dw_cba_backward_full_size_k7(gpu):
    """LKR's k7 at BASELINE config 3's shape (1 x 64 x 2048^2, G = 16) with the
    default size switch (fused): dx and dW bit for bit equal to the
    stand-alone GroupNorm backward followed by the depthwise backward (same
    terms, same order), dgamma and dbeta bit for bit."""
    import torch
    g = gpu
    N, C, H, W, K, G = 1, 64, 2048, 2048, 7, 16
    assert N * H * W >= g.tune_get(g.TUNE_DW_CBA_MIN)
    print("dw_cba_backward full size 1x64x2048^2 k7", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261203)
    xd = torch.randn((N, C, H, W), generator=gen, device="cuda")
    wd = (torch.rand((C, K, K), generator=gen, device="cuda") * 2 - 1) / K
    gd = torch.rand(C, generator=gen, device="cuda") + 0.5
    bd = 0.1 * torch.randn(C, generator=gen, device="cuda")
    dyd = 1e-2 * torch.randn((N, C, H, W), generator=gen, device="cuda")
    z = g.dw_conv_forward(xd, wd, None, 3)
    _, st = g.gn_silu_forward(z, gd, bd, G, eps=EPS)
    dx, dw, dg, db = g.dw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, 3)
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G)
    ux, uw, _ = g.dw_conv_backward(dz, xd, wd, 3, want_db=False)
    torch.cuda.synchronize()
    assert torch.equal(dg, dg_u) and torch.equal(db, db_u)
    assert torch.equal(dx, ux) and torch.equal(dw, uw)


def test_dw_cba_backward_errors(gpu):
    import torch
    g = gpu
    N, C, H, W, K, G = 1, 8, 32, 32, 3, 2
    t = lambda *s: torch.zeros(s, dtype=torch.float32, device="cuda")
    x, z, dy, w = t(N, C, H, W), t(N, C, H, W), t(N, C, H, W), t(C, K, K)
    st = g.Stats(t(N * G), t(N * G), t(N * G))
    with pytest.raises(g.SoarError):
        g.dw_cba_backward(dy, z, x, w, None, None, st, 3, 1)  # C % G
    need = g.dw_cba_backward_workspace_bytes(N, C, H, W, H, W, K, 1, 1, 1, G)
    small = torch.empty(max(need - 256, 1), dtype=torch.uint8, device="cuda")
    with pytest.raises(g.SoarError):
        g.dw_cba_backward(dy, z, x, w, None, None, st, G, 1, ws=small)
    assert "workspace" in g.last_error()
    L = g.lib()
    host_buf = np.zeros(N * C * H * W, np.float32)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    rc = L.soar_dw_cba_backward(host_buf.ctypes.data, z.data_ptr(), x.data_ptr(), w.data_ptr(),
                                None, None, st.mean.data_ptr(), st.rstd.data_ptr(), None,
                                t(N, C, H, W).data_ptr(), None, None, None, N, C, H, W, H, W, K,
                                1, 1, 1, G, g.GN_SILU, ws.data_ptr(), ws.numel(), None)
    assert rc == g.SOAR_EINVAL and "dy" in g.last_error()
