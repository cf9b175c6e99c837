"""Parity of the fused pointwise CBA backward (soar_pw_cba_backward) through
the C-ABI of libsoar_gn.so.

The fused kernel forms dz, the GroupNorm(+SiLU) input gradient, from z and
dy in registers with the GroupNorm dx pass's arithmetic, and computes the
convolution's dx = W^T dz and dW = sum dz x^T from it without storing dz.
Each case checks, on the same device forward:
  dz:      the unfused device GroupNorm backward (soar_gn_silu_backward, whose
           dz the fused kernel reproduces) against the float64 oracle at the
           GroupNorm bar |d| <= 1e-4 (1 + |truth|);
  dx, dW:  against the float64 convolution backward of that device dz, at the
           fp32 bound of their sums (test_gpu_pw_conv.bwd_bounds), so a wrong
           dz inside the fused kernel (a coefficient, a row, a pixel) fails;
  dgamma, dbeta: bit for bit equal to the unfused GroupNorm backward (the
           same reduction and finish run first);
and the fused result against the unfused entry-point path (TUNE_PW_CBA_MIN
= 0) within those bounds.
"""
import numpy as np
import pytest

from test_gpu_parity import EPS, dev, host
from test_gpu_pw_conv import bwd_bounds

pytestmark = pytest.mark.gpu


@pytest.fixture
def fused(gpu):
    """Runs a test with the fused kernel enabled for every size, and the
    stand-alone GroupNorm backward on its multi-kernel path (no one-launch
    small-unit kernel, no folded finish), whose reduction, finish and dx
    arithmetic the fused path shares, so their dz and parameter gradients
    are the same bit for bit."""
    keys = (gpu.TUNE_PW_CBA_MIN, gpu.TUNE_PW_CBA_BLOCKS, gpu.TUNE_SMALL_UNIT,
            gpu.TUNE_FOLD_MAX)
    old = {k: gpu.tune_get(k) for k in keys}
    gpu.tune(gpu.TUNE_PW_CBA_MIN, 1)
    gpu.tune(gpu.TUNE_SMALL_UNIT, 0)
    gpu.tune(gpu.TUNE_FOLD_MAX, 0)
    yield gpu
    for k, v in old.items():
        gpu.tune(k, v)


def _inputs(seed, N, C_in, C_out, HW, kind="normal"):
    r = np.random.default_rng(seed)
    if kind == "offset":
        # z = W x with x = 1e3 + N(0, 1e-2): |mean| >> std in every group
        x = (1e3 + 1e-2 * r.standard_normal((N, C_in, HW))).astype(np.float32)
    else:
        x = r.standard_normal((N, C_in, HW)).astype(np.float32)
    w = (r.uniform(-1.0, 1.0, (C_out, C_in)) / np.sqrt(C_in)).astype(np.float32)
    gm = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    bt = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    dy = (1e-2 * r.standard_normal((N, C_out, HW))).astype(np.float32)
    return x, w, gm, bt, dy


def _within(got, truth, bound, name):
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - np.asarray(truth).reshape(-1))
    ratio = err / (np.asarray(bound).reshape(-1) + 1e-30)
    i = int(np.argmax(ratio))
    assert ratio[i] <= 1.0, f"{name}: err {err[i]:.3e} > bound {np.asarray(bound).reshape(-1)[i]:.3e} at {i}"


CASES = [
    # (N, C_in, C_out, HW, G, silu, kind)
    (1, 64, 64, 4096, 16, True, "normal"),    # one 64 x 64 tile, TM = TN = 2
    (2, 32, 48, 2500, 8, True, "normal"),     # partial row tile, ragged last step
    (1, 16, 24, 1028, 4, False, "normal"),    # no SiLU, TM = TN = 1
    (1, 24, 8, 4100, 2, True, "normal"),      # C_out = 8: rows 8..31 of the tile are zero
    (3, 40, 64, 1000, 16, True, "normal"),    # three samples, partial x tile
    (1, 64, 24, 2048, 4, True, "normal"),     # TM = 1, TN = 2
    (1, 64, 20, 2048, 4, True, "normal"),     # C_out % 8 != 0: the unfused calls
    (1, 8, 64, 516, 32, True, "normal"),      # TM = 2, TN = 1, one 4-pixel lane past a step
    (1, 32, 32, 4096, 8, True, "offset"),     # large mean offset: the mean residual
    (1, 32, 32, 4096, 8, False, "offset"),
]


@pytest.mark.parametrize("N,C_in,C_out,HW,G,silu,kind", CASES)
def test_pw_cba_backward_matches_oracle(fused, oracle, N, C_in, C_out, HW, G, silu, kind):
    g = fused
    print(f"pw_cba_backward N={N} C_in={C_in} C_out={C_out} HW={HW} G={G} silu={silu} {kind}",
          flush=True)
    x, w, gm, bt, dy = _inputs(N * 131 + C_in * 7 + C_out + HW, N, C_in, C_out, HW, kind)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS, silu=silu)
    # the unfused device GroupNorm backward: its dz is what the fused kernel forms
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G, silu=silu)
    dx, dw, dg, db = g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, silu=silu)
    zh, dzh = host(z).astype(np.float32), host(dz).astype(np.float32)

    # dz against the float64 oracle (statistics of the device's own z)
    _, m64, r64 = oracle.gn_silu_fwd_f64(zh, gm, bt, N, C_out, HW, G, EPS, silu=silu,
                                         want_y=False)
    tdz, tdg, tdb = oracle.gn_silu_bwd_f64(dy, zh, gm, bt, m64, r64, N, C_out, HW, G,
                                           silu=silu)
    _within(dzh, tdz, 1e-4 * (1.0 + np.abs(tdz)), "dz")
    _within(host(dg), tdg, 1e-4 * (1.0 + np.abs(tdg)), "dgamma")
    _within(host(db), tdb, 1e-4 * (1.0 + np.abs(tdb)), "dbeta")
    # the parameter gradients come from the same reduction as the unfused path
    assert np.array_equal(host(dg), host(dg_u)) and np.array_equal(host(db), host(db_u))

    # dx, dW against the float64 convolution backward of the device dz
    tx, tw, _ = oracle.conv1x1_bwd_f64(dzh, x, w, N, C_in, C_out, HW, want=("dx", "dw"))
    bx, bw, _ = bwd_bounds(dzh.reshape(N, C_out, HW), x, w)
    _within(host(dx), tx, bx, "dx")
    _within(host(dw), tw, bw, "dW")

    # the unfused entry-point path agrees within the same bounds
    g.tune(g.TUNE_PW_CBA_MIN, 0)
    ux, uw, ug, ub = g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, silu=silu)
    assert np.array_equal(host(ug), host(dg)) and np.array_equal(host(ub), host(db))
    _within(host(ux), tx, bx, "unfused dx")
    _within(host(uw), tw, bw, "unfused dW")


def _launch_names(g, run):
    import torch
    g.prof_summary()
    g.prof_enable(True)
    try:
        out = run()
        torch.cuda.synchronize()
        return out, {r["kernel"] for r in g.prof_summary()}
    finally:
        g.prof_enable(False)


@pytest.mark.parametrize("N,C_in,C_out,HW,G,silu,kind", [CASES[i] for i in (0, 1, 4, 8)])
def test_pw_cba_backward_folded_finish(fused, N, C_in, C_out, HW, G, silu, kind):
    """The GroupNorm backward's finish folded into the fused kernel (every
    block forms its sample's plane and unit sums from the reduction's
    partials; SOAR_TUNE_FOLD_MAX 2048): no finish launch, and dx, dW,
    dgamma, dbeta bit for bit those of the separate finish (0)."""
    g = fused
    print(f"pw_cba_backward folded N={N} C_in={C_in} C_out={C_out} HW={HW} G={G}", flush=True)
    x, w, gm, bt, dy = _inputs(N * 29 + C_in + C_out + HW, N, C_in, C_out, HW, kind)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS, silu=silu)
    runs = {}
    for fold in (0, 2048):
        g.tune(g.TUNE_FOLD_MAX, fold)
        out, names = _launch_names(
            g, lambda: g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, silu=silu))
        assert "pw_cba_bwd" in names, names
        assert ("gn_bwd_finish" in names) == (fold == 0), names
        runs[fold] = [host(t) for t in out]
    for a, b, name in zip(runs[0], runs[2048], ("dx", "dW", "dgamma", "dbeta")):
        assert np.array_equal(a, b), name


@pytest.mark.parametrize("want_dx,want_dw,accumulate", [
    (True, True, True), (True, False, False), (False, True, False), (True, False, True)])
def test_pw_cba_backward_outputs_and_accumulation(fused, oracle, want_dx, want_dw, accumulate):
    """Each output on its own, dx accumulated onto an existing gradient, and
    dW / dgamma / dbeta added to what they hold."""
    g = fused
    N, C_in, C_out, HW, G = 2, 48, 64, 2048, 16
    x, w, gm, bt, dy = _inputs(77, N, C_in, C_out, HW)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS)
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G)
    r = np.random.default_rng(5)
    dx0 = r.standard_normal((N, C_in, HW)).astype(np.float32)
    dw0 = r.standard_normal((C_out, C_in)).astype(np.float32)
    p0 = r.standard_normal(C_out).astype(np.float32)
    dwd = dev(dw0)
    dx, dw, dg, db = g.pw_cba_backward(
        dyd, z, xd, wd, gd, bd, st, G, dx=dev(dx0) if accumulate else None,
        dweight=dwd, dgamma=dev(p0), dbeta=dev(p0), want_dx=want_dx, want_dw=want_dw,
        accumulate_dx=accumulate)
    dzh = host(dz)
    tx, tw, _ = oracle.conv1x1_bwd_f64(dzh, x, w, N, C_in, C_out, HW, want=("dx", "dw"))
    bx, bw, _ = bwd_bounds(dzh, x, w)
    if want_dx:
        t = tx + (dx0.reshape(-1).astype(np.float64) if accumulate else 0.0)
        _within(host(dx), t, bx.reshape(-1) + (2.0 ** -23) * np.abs(t), "dx")
    else:
        assert dx is None
    if want_dw:
        t = tw + dw0.reshape(-1).astype(np.float64)
        _within(host(dw), t, bw.reshape(-1) + (2.0 ** -23) * np.abs(t), "dW")
    else:
        assert dw is None and np.array_equal(host(dwd), dw0)  # not touched
    # dgamma = fp32(p0 + s) with s the float64 sum, the unfused result fp32(s):
    # the two differ by at most the two roundings
    for got, u, name in ((dg, dg_u, "dgamma"), (db, db_u, "dbeta")):
        u = host(u).astype(np.float64)
        t = p0.astype(np.float64) + u
        _within(host(got), t, 2.0 ** -24 * (np.abs(u) + np.abs(t)) + 1e-30, name)


def test_pw_cba_backward_params_alone_in_queried_workspace(fused):
    """dgamma / dbeta alone run the GroupNorm backward only, within the
    workspace the size query returns (the fused path's, smaller than dz),
    bit for bit the full call's."""
    import torch
    g = fused
    N, C_in, C_out, HW, G = 1, 32, 64, 4096, 8
    x, w, gm, bt, dy = _inputs(41, N, C_in, C_out, HW)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS)
    need = g.pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G)
    assert 0 < need < N * C_out * HW * 4
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    _, _, fg, fb = g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, ws=ws)
    _, _, pg, pb = g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G, want_dx=False,
                                     want_dw=False, ws=ws)
    assert np.array_equal(host(pg), host(fg)) and np.array_equal(host(pb), host(fb))


def test_pw_cba_backward_block_counts_agree(fused):
    """The pixel chunking (TUNE_PW_CBA_BLOCKS) changes only the order of the
    weight gradient's partial sums; dx is the same bit for bit."""
    g = fused
    N, C_in, C_out, HW, G = 1, 64, 64, 1 << 16, 16
    x, w, gm, bt, dy = _inputs(3, N, C_in, C_out, HW)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS)
    outs = []
    for blocks in (64, 256, 1024):
        g.tune(g.TUNE_PW_CBA_BLOCKS, blocks)
        outs.append([host(t) for t in g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G)])
    for o in outs[1:]:
        assert np.array_equal(o[0], outs[0][0])  # dx
        assert np.allclose(o[1], outs[0][1], rtol=1e-5, atol=1e-5 * np.abs(outs[0][1]).max())
        assert np.array_equal(o[2], outs[0][2]) and np.array_equal(o[3], outs[0][3])
    # and two runs of one setting agree bit for bit
    again = [host(t) for t in g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G)]
    for a, b in zip(again, outs[-1]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("N,C_in,C_out,HW,G,accumulate", [
    (3, 40, 48, 2048, 8, False),   # TM = TN = 2: rows 40..63 of x/dx, 48..63 of z/dy past the end
    (3, 40, 48, 2048, 8, True),    # dx read back and added to (the same rows)
    (2, 24, 40, 1028, 4, False),   # TN = 1: rows 24..31 of dx past the end
])
def test_pw_cba_backward_tile_rows_stay_in_their_sample(fused, oracle, N, C_in, C_out, HW, G,
                                                        accumulate):
    """Tile rows past C_in / C_out neither read nor write outside their own
    sample: dy, z, x and dx sit at the start of larger buffers whose tails
    hold a sentinel (NaN behind the inputs, so a row read past the last
    sample's z or dy would turn dx into NaN; a finite marker behind dx,
    which must stay bit for bit), and dx of every sample, the first rows of
    samples 1.. included, matches the float64 convolution backward of the
    unfused dz."""
    import torch
    g = fused
    print(f"pw_cba_backward sentinel tails N={N} C_in={C_in} C_out={C_out} HW={HW} G={G} "
          f"acc={accumulate}", flush=True)
    # the fused kernel takes the shape: its workspace holds no dz
    assert g.pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G) < N * C_out * HW * 4
    x, w, gm, bt, dy = _inputs(N * 7 + C_in + 3 * C_out, N, C_in, C_out, HW)
    xd, wd, gd, bd, dyd = dev(x), dev(w), dev(gm), dev(bt), dev(dy)
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS)
    dz, _, _ = g.gn_silu_backward(dyd, z, gd, bd, st, G)
    tail = 64 * HW  # more than any tile's rows past the last sample

    def in_big(t, fill):
        n = t.numel()
        big = torch.full((n + tail,), fill, dtype=torch.float32, device="cuda")
        big[:n].copy_(t.reshape(-1))
        return big, big[:n].view(t.shape)

    _, dyv = in_big(dyd, float("nan"))
    _, zv = in_big(z, float("nan"))
    _, xv = in_big(xd, float("nan"))
    dx0 = np.random.default_rng(9).standard_normal((N, C_in, HW)).astype(np.float32)
    dxb, dxv = in_big(dev(dx0) if accumulate else torch.zeros((N, C_in, HW), device="cuda"),
                      12345.0)
    dx, _, _, _ = g.pw_cba_backward(dyv, zv, xv, wd, gd, bd, st, G, dx=dxv, want_dw=False,
                                    accumulate_dx=accumulate)
    torch.cuda.synchronize()
    assert dx.data_ptr() == dxb.data_ptr()
    assert bool((dxb[N * C_in * HW:] == 12345.0).all()), "dx stores past the last sample"
    dzh = host(dz)
    tx, _, _ = oracle.conv1x1_bwd_f64(dzh, x, w, N, C_in, C_out, HW, want=("dx",))
    bx, _, _ = bwd_bounds(dzh, x, w)
    t = tx + (dx0.reshape(-1).astype(np.float64) if accumulate else 0.0)
    _within(host(dx), t, bx.reshape(-1) + (2.0 ** -23) * np.abs(t), "dx")


def test_pw_cba_backward_full_size(gpu):
    """BASELINE config 3's shape behind a 64 -> 64 pointwise conv (the
    default size switch takes the fused kernel): dx at 200000 sampled
    entries and all of dW against float64 sums of the device dz, dgamma and
    dbeta bit for bit against the unfused GroupNorm backward."""
    import torch
    g = gpu
    N, C_in, C_out, HW, G = 1, 64, 64, 2048 * 2048, 16
    assert N * HW >= g.tune_get(g.TUNE_PW_CBA_MIN)
    print("pw_cba_backward full size 1x64x2048^2 G=16", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261202)
    xd = torch.randn((N, C_in, HW), generator=gen, device="cuda")
    wd = (torch.rand((C_out, C_in), generator=gen, device="cuda") * 2 - 1) / 8.0
    gd = torch.rand(C_out, generator=gen, device="cuda") + 0.5
    bd = 0.1 * torch.randn(C_out, generator=gen, device="cuda")
    dyd = 1e-2 * torch.randn((N, C_out, HW), generator=gen, device="cuda")
    z, _, st = g.pw_conv_gn_silu_forward(xd, wd, None, gd, bd, G, eps=EPS)
    dz, dg_u, db_u = g.gn_silu_backward(dyd, z, gd, bd, st, G)
    dx, dw, dg, db = g.pw_cba_backward(dyd, z, xd, wd, gd, bd, st, G)
    torch.cuda.synchronize()
    assert torch.equal(dg, dg_u) and torch.equal(db, db_u)
    # dW in float64 on the device (test-side reference of the same dz)
    dz64, x64 = dz[0].double(), xd[0].double()
    tw = dz64 @ x64.T
    mw = dz64.abs() @ x64.abs().T
    bw = (N * HW + 2) * 2.0 ** -24 * mw
    assert bool(((dw.double() - tw).abs() <= bw).all()), float(((dw.double() - tw).abs() / bw).max())
    # dx at sampled pixels
    idx = torch.randint(0, HW, (200000,), generator=gen, device="cuda")
    w64 = wd.double()
    tx = w64.T @ dz64[:, idx]
    bx = (C_out + 2) * 2.0 ** -24 * (w64.abs().T @ dz64[:, idx].abs())
    got = dx[0][:, idx].double()
    assert bool(((got - tx).abs() <= bx).all()), float(((got - tx).abs() / bx).max())


def test_pw_cba_backward_errors(gpu):
    import torch
    g = gpu
    N, C_in, C_out, HW, G = 1, 16, 16, 4096, 4
    t = lambda *s: torch.zeros(s, dtype=torch.float32, device="cuda")
    x, w, z, dy = t(N, C_in, HW), t(C_out, C_in), t(N, C_out, HW), t(N, C_out, HW)
    st = g.Stats(t(N * G), t(N * G), t(N * G))
    ws_need = g.pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G)
    small = torch.empty(max(ws_need - 256, 1), dtype=torch.uint8, device="cuda")
    with pytest.raises(g.SoarError):
        g.pw_cba_backward(dy, z, x, w, None, None, st, G, ws=small)
    assert "workspace" in g.last_error()
    with pytest.raises(g.SoarError):
        g.pw_cba_backward(dy, z, x, w, None, None, st, 3)  # C % G
    # a host pointer is an error status, not a fault
    L = g.lib()
    host_buf = np.zeros(N * C_out * HW, np.float32)
    ws = torch.empty(ws_need, dtype=torch.uint8, device="cuda")
    rc = L.soar_pw_cba_backward(host_buf.ctypes.data, z.data_ptr(), x.data_ptr(), w.data_ptr(),
                                None, None, st.mean.data_ptr(), st.rstd.data_ptr(), None,
                                t(N, C_in, HW).data_ptr(), None, None, None, N, C_in, C_out, HW,
                                G, g.GN_SILU, ws.data_ptr(), ws.numel(), None)
    assert rc == g.SOAR_EINVAL and "dy" in g.last_error()
