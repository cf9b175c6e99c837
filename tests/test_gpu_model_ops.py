"""The model operators of include/soar_ops.h on the MI355X, one by one,
through the C-ABI, against float64 statements of the reference's formulas.

Bars: index permutations (pixel shuffle, pad, crop, fill) bit-exact;
elementwise fp32 formulas within a few ulps of float64; reductions
(conv, pooling, loss sums, norms) within (K+2) * 2^-24 * sum|terms| for a
K-term sum; AdamW bit-exact against scalar fp32 (numpy) arithmetic.
Backward entry points add into their outputs, so every gradient buffer is
pre-filled with a known value and the test checks output - prefill.
"""
import ctypes

import numpy as np
import pytest

import soar_model_ref as smr

pytestmark = pytest.mark.gpu

F32 = np.float32
U32 = 2.0 ** -24


@pytest.fixture(scope="module")
def env():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import soar_gn
    soar_gn.lib()
    return soar_gn, torch


def dev(torch, a):
    return torch.tensor(np.ascontiguousarray(a, dtype=F32), device="cuda")


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def host(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ok(gn, rc):
    assert rc == 0, gn.last_error()


# ---- general grouped convolution ---------------------------------------------
def conv_ref(x, w, b, S, pad, D, G):
    """float64 direct convolution (and the magnitudes for the bound)."""
    N, Ci, H, W = x.shape
    Co, cig, K, _ = w.shape
    Ho = (H + 2 * pad - D * (K - 1) - 1) // S + 1
    Wo = (W + 2 * pad - D * (K - 1) - 1) // S + 1
    xp = np.zeros((N, Ci, H + 2 * pad, W + 2 * pad))
    xp[:, :, pad:pad + H, pad:pad + W] = x
    y = np.zeros((N, Co, Ho, Wo))
    mag = np.zeros_like(y)
    cog = Co // G
    for co in range(Co):
        g = co // cog
        for q in range(cig):
            for ky in range(K):
                for kx in range(K):
                    sl = xp[:, g * cig + q, ky * D: ky * D + S * (Ho - 1) + 1: S,
                            kx * D: kx * D + S * (Wo - 1) + 1: S]
                    y[:, co] += w[co, q, ky, kx] * sl
                    mag[:, co] += abs(w[co, q, ky, kx]) * np.abs(sl)
    if b is not None:
        y += b[None, :, None, None]
        mag += np.abs(b)[None, :, None, None]
    return y, mag


@pytest.mark.parametrize("N,Ci,Co,H,W,K,S,D,G,bias", [
    (1, 1, 16, 64, 64, 3, 2, 1, 1, False),   # the model's stem
    (2, 3, 16, 33, 47, 3, 2, 1, 1, True),    # odd sizes, RGB stem
    (1, 1, 16, 1024, 1024, 3, 2, 1, 1, False),  # the stem at 1024^2: 512 dW chunks
    (1, 4, 12, 40, 36, 1, 1, 1, 1, True),    # K = 1, C_out in tiles of 4
    (2, 2, 8, 50, 30, 3, 1, 1, 1, True),     # stride 1, C_out 8
    (1, 8, 12, 20, 18, 3, 1, 2, 4, True),    # grouped, dilated
    (1, 6, 6, 11, 9, 5, 3, 1, 2, False),     # stride 3, K 5
])
def test_general_conv(env, N, Ci, Co, H, W, K, S, D, G, bias):
    gn, torch = env
    print(f"case: conv N={N} {Ci}->{Co} {H}x{W} K={K} S={S} D={D} G={G}", flush=True)
    r = np.random.default_rng(H * W + K)
    pad = smr.autopad(K, -1, D)
    x = r.normal(size=(N, Ci, H, W)).astype(F32)
    w = r.uniform(-0.5, 0.5, size=(Co, Ci // G, K, K)).astype(F32)
    b = r.normal(size=Co).astype(F32) if bias else None
    y_ref, mag = conv_ref(x.astype(np.float64), w.astype(np.float64),
                          None if b is None else b.astype(np.float64), S, pad, D, G)
    Ho, Wo = y_ref.shape[2:]
    L = gn.lib()
    xd, wd = dev(torch, x), dev(torch, w)
    bd = dev(torch, b) if bias else None
    yd = torch.empty((N, Co, Ho, Wo), device="cuda")
    ok(gn, L.soar_conv_forward(P(xd), P(wd), P(bd) if bias else None, P(yd), N, Ci, Co, H, W,
                               Ho, Wo, K, pad, S, D, G, None))
    nterm = Ci // G * K * K + 2
    assert np.all(np.abs(host(torch, yd) - y_ref) <= nterm * U32 * mag + 1e-30)
    # backward: the adjoint identities against float64 and a direct dW
    dy = r.normal(size=(N, Co, Ho, Wo)).astype(F32)
    dyd = dev(torch, dy)
    dx = torch.full((N, Ci, H, W), 0.25, device="cuda")
    dw = torch.full(w.shape, -1.0, device="cuda")
    db = torch.full((Co,), 2.0, device="cuda")
    wsb = L.soar_conv_backward_workspace_bytes(N, Ci, Co, H, W, Ho, Wo, K, pad, S, D, G)
    ws = torch.empty(max(wsb, 8), dtype=torch.uint8, device="cuda")
    ok(gn, L.soar_conv_backward(P(dyd), P(xd), P(wd), P(dx), P(dw), P(db), N, Ci, Co, H, W, Ho,
                                Wo, K, pad, S, D, G, gn.GN_ACCUMULATE_DX, P(ws), wsb, None))
    dxh = host(torch, dx).astype(np.float64) - 0.25
    dwh = host(torch, dw).astype(np.float64) + 1.0
    dbh = host(torch, db).astype(np.float64) - 2.0
    # <conv(x), dy> = <x, dx> + <b, db> identities, each term in float64
    y0, _ = conv_ref(x.astype(np.float64), w.astype(np.float64), None, S, pad, D, G)
    lhs = float(np.sum(y0 * dy))
    assert abs(float(np.sum(x * dxh)) - lhs) <= 1e-4 * np.sum(np.abs(y0 * dy))
    assert abs(float(np.sum(w * dwh)) - lhs) <= 1e-4 * np.sum(np.abs(y0 * dy))
    np.testing.assert_allclose(dbh, dy.astype(np.float64).sum(axis=(0, 2, 3)), rtol=1e-5,
                               atol=1e-4)
    # dW directly: dW[co,q,ky,kx] = sum dy * shifted x (float64)
    xp = np.zeros((N, Ci, H + 2 * pad, W + 2 * pad))
    xp[:, :, pad:pad + H, pad:pad + W] = x
    cog = Co // G
    for co in (0, Co - 1):
        for q in range(Ci // G):
            ci = (co // cog) * (Ci // G) + q
            for ky in range(K):
                for kx in range(K):
                    sl = xp[:, ci, ky * D: ky * D + S * (Ho - 1) + 1: S,
                            kx * D: kx * D + S * (Wo - 1) + 1: S]
                    t = float(np.sum(dy[:, co] * sl))
                    m = float(np.sum(np.abs(dy[:, co] * sl)))
                    assert abs(dwh[co, q, ky, kx] - t) <= (N * Ho * Wo + 3) * U32 * m + 1e-6


def dw_ones(x):
    """dW of the stem conv (16 outputs, k3 s2 p1) for dy = 1: per tap, the
    sum of the input pixels that tap reads."""
    xp = np.zeros((34, 34))
    xp[1:33, 1:33] = x[0, 0]
    t = np.array([[xp[ky:ky + 31:2, kx:kx + 31:2].sum() for kx in range(3)] for ky in range(3)])
    return np.broadcast_to(t, (16, 1, 3, 3))


def test_conv_reference_signature(env):
    """soar_conv2d_forward/backward (one sample, library workspace, all
    gradients added)."""
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(5)
    x = r.normal(size=(1, 1, 32, 32)).astype(F32)
    w = r.uniform(-0.5, 0.5, size=(16, 1, 3, 3)).astype(F32)
    y_ref, mag = conv_ref(x.astype(np.float64), w.astype(np.float64), None, 2, 1, 1, 1)
    xd, wd = dev(torch, x), dev(torch, w)
    yd = torch.empty((16, 16, 16), device="cuda")
    ok(gn, L.soar_conv2d_forward(P(xd), P(wd), None, P(yd), 1, 16, 32, 32, 16, 16, 3, 1, 2, 1, 1,
                                 None))
    assert np.all(np.abs(host(torch, yd) - y_ref[0]) <= 11 * U32 * mag[0] + 1e-30)
    dy = dev(torch, np.ones((16, 16, 16), F32))
    dx = torch.zeros((1, 32, 32), device="cuda")
    dw = torch.zeros((16, 1, 3, 3), device="cuda")
    ok(gn, L.soar_conv2d_backward(P(dy), P(xd), P(wd), P(dx), P(dw), None, 1, 16, 32, 32, 16, 16,
                                  3, 1, 2, 1, 1, None))
    ok(gn, L.soar_conv2d_backward(P(dy), P(xd), P(wd), P(dx), P(dw), None, 1, 16, 32, 32, 16, 16,
                                  3, 1, 2, 1, 1, None))
    # two calls add twice; with dy = 1, dx at an input pixel is the sum of
    # the taps that reach it: at stride 2 / pad 1, rows and columns 5 are
    # reached by taps 0 and 2, rows and columns 4 by tap 1 only
    dx1 = host(torch, dx) / 2
    assert abs(float(dx1[0, 5, 5]) - float(w[:, 0, ::2, ::2].sum())) < 1e-5
    assert abs(float(dx1[0, 4, 4]) - float(w[:, 0, 1, 1].sum())) < 1e-5
    np.testing.assert_allclose(host(torch, dw) / 2, dw_ones(x), rtol=1e-5, atol=1e-4)


# ---- elementwise / per-plane -------------------------------------------------------
def test_sigmoid_convex_broadcast_pool(env):
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(6)
    n = 10007
    x = (r.normal(size=n) * 8).astype(F32)
    xd, yd = dev(torch, x), torch.empty(n, device="cuda")
    ok(gn, L.soar_sigmoid_forward(P(xd), P(yd), n, None))
    y = host(torch, yd)
    yt = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.all(np.abs(y - yt) <= 4 * U32 * yt + 1e-38)
    gy = r.normal(size=n).astype(F32)
    gx = torch.full((n,), 1.0, device="cuda")
    ok(gn, L.soar_sigmoid_backward(P(dev(torch, gy)), P(yd), P(gx), n, None))
    gxt = 1.0 + gy * y.astype(np.float64) * (1.0 - y)
    np.testing.assert_allclose(host(torch, gx), gxt, rtol=1e-6, atol=1e-7)

    a, b, g = (r.normal(size=n).astype(F32) for _ in range(3))
    ad, bd, gd = dev(torch, a), dev(torch, b), dev(torch, g)
    ok(gn, L.soar_convex_combination_forward(P(gd), P(ad), P(bd), P(yd), n, None))
    np.testing.assert_allclose(host(torch, yd), g.astype(np.float64) * a + (1 - g.astype(np.float64)) * b,
                               rtol=1e-6, atol=1e-6)
    ga, gb, gg = (torch.zeros(n, device="cuda") for _ in range(3))
    ok(gn, L.soar_convex_combination_backward(P(dev(torch, gy)), P(gd), P(ad), P(bd), P(gg), P(ga),
                                              P(gb), n, None))
    np.testing.assert_allclose(host(torch, ga), gy * g.astype(np.float64), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(host(torch, gb), gy * (1 - g.astype(np.float64)), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(host(torch, gg), gy * (a.astype(np.float64) - b), rtol=1e-6, atol=1e-6)

    C, HW = 37, 1023
    A = r.normal(size=(C, HW)).astype(F32)
    B = r.normal(size=C).astype(F32)
    Ad, Bd, Yd = dev(torch, A), dev(torch, B), torch.empty((C, HW), device="cuda")
    ok(gn, L.soar_mul_broadcast_forward(P(Ad), P(Bd), P(Yd), C, HW, None))
    np.testing.assert_array_equal(host(torch, Yd), A * B[:, None])
    GY = r.normal(size=(C, HW)).astype(F32)
    GA, GB = torch.zeros((C, HW), device="cuda"), torch.full((C,), 3.0, device="cuda")
    ok(gn, L.soar_mul_broadcast_backward(P(dev(torch, GY)), P(Ad), P(Bd), P(GA), P(GB), C, HW, None))
    np.testing.assert_array_equal(host(torch, GA), GY * B[:, None])
    gbt = (GY.astype(np.float64) * A).sum(axis=1)
    assert np.all(np.abs(host(torch, GB) - 3.0 - gbt) <= 4 * U32 * (np.abs(GY * A).sum(axis=1) + 3))

    pooled = torch.empty(C, device="cuda")
    ok(gn, L.soar_global_avg_pool_forward(P(Ad), P(pooled), C, HW, None))
    np.testing.assert_allclose(host(torch, pooled), A.astype(np.float64).mean(axis=1), rtol=1e-6,
                               atol=1e-7)
    gi = torch.zeros((C, HW), device="cuda")
    ok(gn, L.soar_global_avg_pool_backward(P(Bd), P(gi), C, HW, None))
    np.testing.assert_allclose(host(torch, gi), np.broadcast_to((B / F32(HW))[:, None], (C, HW)),
                               rtol=1e-7)


@pytest.mark.parametrize("acc", [0, 1])
def test_sigmoid_gates_match_separate_ops(env, acc):
    """soar_sigmoid_convex_* and soar_mul_sigmoid_broadcast_* (the Fuse / Ctx
    gates with the sigmoid folded in) give bit for bit the values of
    soar_sigmoid_forward followed by the gate's own entry point, and the
    gradients of the gate's backward followed by soar_sigmoid_backward,
    written (flags 0) or added (SOAR_GN_ACCUMULATE_DX); and match float64."""
    gn, torch = env
    L = gn.lib()
    fl = gn.GN_ACCUMULATE_DX if acc else 0
    print(f"case: sigmoid gates acc={acc}", flush=True)
    r = np.random.default_rng(16 + acc)
    n = 20011
    z, a, b, gy = ((r.normal(size=n) * s).astype(F32) for s in (4, 1, 1, 1))
    zd, ad, bd, gyd = dev(torch, z), dev(torch, a), dev(torch, b), dev(torch, gy)
    # separate: s = sigmoid(z), then the convex combination
    sd, y0 = torch.empty(n, device="cuda"), torch.empty(n, device="cuda")
    ok(gn, L.soar_sigmoid_forward(P(zd), P(sd), n, None))
    ok(gn, L.soar_convex_combination_forward(P(sd), P(ad), P(bd), P(y0), n, None))
    y1 = torch.empty(n, device="cuda")
    ok(gn, L.soar_sigmoid_convex_forward(P(zd), P(ad), P(bd), P(y1), n, None))
    np.testing.assert_array_equal(host(torch, y1), host(torch, y0))
    s64 = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    yt = s64 * a + (1 - s64) * b
    assert np.all(np.abs(host(torch, y1) - yt) <= 8 * U32 * (np.abs(a) + np.abs(b)) + 1e-30)
    base = [r.normal(size=n).astype(F32) for _ in range(3)] if acc else [np.zeros(n, F32)] * 3
    gs, ga0, gb0, gz0 = (torch.zeros(n, device="cuda") for _ in range(4))
    ga0.copy_(dev(torch, base[1]))
    gb0.copy_(dev(torch, base[2]))
    gz0.copy_(dev(torch, base[0]))
    # (the gate's own gradient, fresh, then through the sigmoid into gz0)
    ok(gn, L.soar_convex_combination_backward_ex(P(gyd), P(sd), P(ad), P(bd), None, P(ga0),
                                                 P(gb0), n, fl, None))
    ok(gn, L.soar_convex_combination_backward_ex(P(gyd), P(sd), P(ad), P(bd), P(gs), None,
                                                 None, n, 0, None))
    ok(gn, L.soar_sigmoid_backward_ex(P(gs), P(sd), P(gz0), n, fl, None))
    ga1, gb1, gz1 = (dev(torch, base[k]) for k in (1, 2, 0))
    ok(gn, L.soar_sigmoid_convex_backward_ex(P(gyd), P(zd), P(ad), P(bd), P(gz1), P(ga1),
                                             P(gb1), n, fl, None))
    for got, want, name in ((ga1, ga0, "grad_a"), (gb1, gb0, "grad_b"), (gz1, gz0, "grad_z")):
        np.testing.assert_array_equal(host(torch, got), host(torch, want), err_msg=name)
    gzt = base[0] + gy * (a.astype(np.float64) - b) * s64 * (1 - s64)
    np.testing.assert_allclose(host(torch, gz1), gzt, rtol=1e-5, atol=1e-6)

    C, HW = 37, 1023
    A = r.normal(size=(C, HW)).astype(F32)
    Z = (r.normal(size=C) * 3).astype(F32)
    GY = r.normal(size=(C, HW)).astype(F32)
    Ad, Zd, GYd = dev(torch, A), dev(torch, Z), dev(torch, GY)
    Sd, Y0, Y1 = torch.empty(C, device="cuda"), torch.empty((C, HW), device="cuda"), \
        torch.empty((C, HW), device="cuda")
    ok(gn, L.soar_sigmoid_forward(P(Zd), P(Sd), C, None))
    ok(gn, L.soar_mul_broadcast_forward(P(Ad), P(Sd), P(Y0), C, HW, None))
    ok(gn, L.soar_mul_sigmoid_broadcast_forward(P(Ad), P(Zd), P(Y1), C, HW, None))
    np.testing.assert_array_equal(host(torch, Y1), host(torch, Y0))
    ga_base = r.normal(size=(C, HW)).astype(F32) if acc else np.zeros((C, HW), F32)
    gz_base = r.normal(size=C).astype(F32) if acc else np.zeros(C, F32)
    GA0, GS, GZ0 = dev(torch, ga_base), torch.zeros(C, device="cuda"), dev(torch, gz_base)
    ok(gn, L.soar_mul_broadcast_backward_ex(P(GYd), P(Ad), P(Sd), P(GA0), P(GS), C, HW, fl,
                                            None))
    GS0 = torch.zeros(C, device="cuda")
    ok(gn, L.soar_mul_broadcast_backward_ex(P(GYd), P(Ad), P(Sd), None, P(GS0), C, HW, 0, None))
    ok(gn, L.soar_sigmoid_backward_ex(P(GS0), P(Sd), P(GZ0), C, fl, None))
    GA1, GZ1 = dev(torch, ga_base), dev(torch, gz_base)
    ok(gn, L.soar_mul_sigmoid_broadcast_backward_ex(P(GYd), P(Ad), P(Zd), P(GA1), P(GZ1), C, HW,
                                                    fl, None))
    np.testing.assert_array_equal(host(torch, GA1), host(torch, GA0))
    np.testing.assert_array_equal(host(torch, GZ1), host(torch, GZ0))
    s64 = 1.0 / (1.0 + np.exp(-Z.astype(np.float64)))
    gzt = gz_base + (GY.astype(np.float64) * A).sum(axis=1) * s64 * (1 - s64)
    np.testing.assert_allclose(host(torch, GZ1), gzt, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("C,H,W,Ho,Wo", [(3, 2, 2, 4, 4), (5, 4, 4, 16, 16), (2, 7, 5, 14, 10),
                                         (2, 6, 9, 9, 13), (1, 32, 32, 64, 64),
                                         (2, 16, 12, 5, 7), (2, 3, 3, 24, 24), (2, 3, 2, 40, 37),
                                         (2, 4, 8, 16, 16), (16, 16, 16, 32, 32), (3, 1, 1, 4, 6),
                                         (2, 9, 70, 18, 140), (1, 3, 130, 11, 260),
                                         (2, 20, 100, 7, 33), (1, 5, 66, 20, 264),
                                         (2, 1, 3, 2, 6), (1, 1, 2, 4, 8), (2, 40, 70, 160, 280)])
def test_upsample(env, C, H, W, Ho, Wo):
    """Forward and the gathered backward against float64 loops of the
    reference's index arithmetic (fp32 source coordinates).  The shapes
    cover the exact 2x and 4x backward (one-pixel sides included), the
    tiled backward at other factors up to 2x and up to 4x (one and several
    64-column tiles, ragged last tiles), the per-pixel backward at 8x and
    larger (column runs longer than its register window), downsampling
    (sources no destination reads) and mixed axis factors."""
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(H * Ho)
    x = r.normal(size=(C, H, W)).astype(F32)
    xd, yd = dev(torch, x), torch.empty((C, Ho, Wo), device="cuda")
    ok(gn, L.soar_upsample_bilinear_forward(P(xd), P(yd), C, H, W, Ho, Wo, None))
    sy, sx = F32(H) / F32(Ho), F32(W) / F32(Wo)

    def taps(sc, d, n):
        f = max(F32(sc * (F32(d) + F32(0.5)) - F32(0.5)), F32(0))
        i0 = min(int(f), n - 1)
        i1 = i0 + (1 if i0 < n - 1 else 0)
        l1 = float(f) - i0
        return i0, i1, 1 - l1, l1

    yt = np.zeros((C, Ho, Wo))
    gt = np.zeros((C, H, W))
    go = r.normal(size=(C, Ho, Wo))
    for y in range(Ho):
        y0, y1, a0, a1 = taps(sy, y, H)
        for xx in range(Wo):
            x0, x1, b0, b1 = taps(sx, xx, W)
            yt[:, y, xx] = (a0 * (b0 * x[:, y0, x0] + b1 * x[:, y0, x1]) +
                            a1 * (b0 * x[:, y1, x0] + b1 * x[:, y1, x1]))
            for (yy, wy) in ((y0, a0), (y1, a1)):
                for (xs, wx) in ((x0, b0), (x1, b1)):
                    gt[:, yy, xs] += wy * wx * go[:, y, xx]
    np.testing.assert_allclose(host(torch, yd), yt, rtol=1e-6, atol=1e-6)
    gi = torch.full((C, H, W), -0.5, device="cuda")
    ok(gn, L.soar_upsample_bilinear_backward(P(dev(torch, go)), P(gi), C, H, W, Ho, Wo, None))
    np.testing.assert_allclose(host(torch, gi) + 0.5, gt, rtol=1e-5, atol=2e-5)


def test_pixel_shuffle_pad_crop(env):
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(7)
    x = r.normal(size=(8, 5, 3)).astype(F32)
    xd, yd = dev(torch, x), torch.empty((2, 10, 6), device="cuda")
    ok(gn, L.soar_pixel_shuffle_forward(P(xd), P(yd), 8, 5, 3, 2, None))
    ref = torch.nn.functional.pixel_shuffle(torch.tensor(x)[None], 2)[0].numpy()
    np.testing.assert_array_equal(host(torch, yd), ref)
    gx = torch.full((8, 5, 3), 1.0, device="cuda")
    ok(gn, L.soar_pixel_shuffle_backward(P(yd), P(gx), 8, 5, 3, 2, None))
    np.testing.assert_array_equal(host(torch, gx), x + F32(1.0))
    assert L.soar_pixel_shuffle_forward(P(xd), P(yd), 6, 5, 3, 2, None) == gn.SOAR_EINVAL

    for (H, W, ph, pw) in ((5, 7, 3, 1), (2, 3, 30, 29)):
        x = r.normal(size=(2, H, W)).astype(F32)
        t = torch.tensor(x[None].astype(np.float64), requires_grad=True)
        pt = smr.pad_spatial(t, ph, pw)
        xd = dev(torch, x)
        out = torch.empty((2, H + ph, W + pw), device="cuda")
        ok(gn, L.soar_pad_spatial_forward(P(xd), P(out), 2, H, W, ph, pw, None))
        np.testing.assert_array_equal(host(torch, out), pt.detach().numpy()[0].astype(F32))
        go = r.normal(size=(2, H + ph, W + pw)).astype(F32)
        pt.backward(torch.tensor(go[None].astype(np.float64)))
        gi = torch.zeros((2, H, W), device="cuda")
        ok(gn, L.soar_pad_spatial_backward(P(dev(torch, go)), P(gi), 2, H, W, ph, pw, None))
        np.testing.assert_allclose(host(torch, gi), t.grad.numpy()[0], rtol=1e-6, atol=1e-6)
        crop = torch.empty((2, H, W), device="cuda")
        ok(gn, L.soar_unpad_spatial_forward(P(out), P(crop), 2, H + ph, W + pw, H, W, None))
        np.testing.assert_array_equal(host(torch, crop), x)
        gp = torch.full((2, H + ph, W + pw), 1.0, device="cuda")
        ok(gn, L.soar_unpad_spatial_backward(P(xd), P(gp), 2, H + ph, W + pw, H, W, None))
        exp = np.ones((2, H + ph, W + pw), F32)
        exp[:, :H, :W] += x
        np.testing.assert_array_equal(host(torch, gp), exp)


# ---- losses ------------------------------------------------------------------------
def test_losses(env):
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(8)
    n = 64 * 64
    z = (r.normal(size=n) * 3).astype(F32)
    y = (r.uniform(size=n) < 0.3).astype(F32)
    zd, yd = dev(torch, z), dev(torch, y)
    out = (ctypes.c_float * 6)()
    ok(gn, L.soar_dice_bce_loss_forward(P(zd), P(yd), n, 1.0, 0.5, 0.5, 3.0, 1.0, out, None))
    lo = smr.dice_bce_forward(z, y)
    vals = list(out)
    for got, want in zip(vals, (lo.total, lo.bce, lo.dice, lo.inter, lo.sum_p, lo.sum_y)):
        assert abs(got - want) <= 2e-6 * abs(want) + 1e-7, (got, want)
    f = ctypes.c_float()
    ok(gn, L.soar_bce_with_logits_forward(P(zd), P(yd), 2.0, 3.0, n, ctypes.byref(f), None))
    assert abs(f.value - 2 * lo.bce) <= 2e-6 * lo.bce
    # (gradients are ~1e-6 here: accumulate onto zeros, then a second call
    # doubles them, rather than subtract a large prefill)
    gz = torch.zeros(n, device="cuda")
    ok(gn, L.soar_dice_bce_loss_backward(P(zd), P(yd), P(gz), 1.0, 1.0, 0.5, 0.5, 3.0, 1.0,
                                         vals[3], vals[4], vals[5], n, None))
    st = smr.LossOut(0, 0, 0, vals[3], vals[4], vals[5])
    g = smr.dice_bce_grad(z, y, st)
    # fp32 bound of the reference's formula (loss_kernels.cu:234-246): its
    # sums cancel (3*sig - 3 as sig -> 1, 2y*denom - numer), so the bound
    # is in the magnitudes of their terms
    z64, y64 = z.astype(np.float64), y.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-z64))
    denom = st.sum_p + st.sum_y + 1.0
    numer = 2.0 * st.inter + 1.0
    mag = ((sig * (1 + 2 * y64) + 3 * y64) * 0.5 / n +
           0.5 * (2 * y64 * denom + numer) / denom ** 2 * sig * (1 - sig))
    g1 = host(torch, gz)
    assert np.all(np.abs(g1 - g) <= 16 * U32 * mag)
    ok(gn, L.soar_dice_bce_loss_backward(P(zd), P(yd), P(gz), 1.0, 1.0, 0.5, 0.5, 3.0, 1.0,
                                         vals[3], vals[4], vals[5], n, None))
    np.testing.assert_array_equal(host(torch, gz), g1 + g1)
    p = torch.empty(n, device="cuda")
    m = torch.empty(n, dtype=torch.uint8, device="cuda")
    ok(gn, L.soar_sigmoid_threshold(P(zd), P(p), P(m), n, 0.5, None))
    pt = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    np.testing.assert_allclose(host(torch, p), pt, rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(host(torch, m), (z >= 0).astype(np.uint8))


# ---- channel concatenation -----------------------------------------------------------
@pytest.mark.parametrize("N,HW", [(2, 7), (2, 16), (1, 4096), (3, 1)])
def test_concat_channels(env, N, HW):
    """One-launch concatenation: forward bit-exact against np.concatenate;
    backward writes (NaN prefill), adds (flags), and skips NULL pieces."""
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(N * HW)
    chans = [3, 5, 2, 8]
    K = len(chans)
    xs = [r.normal(size=(N, c, HW)).astype(F32) for c in chans]
    xd = [dev(torch, x) for x in xs]
    out = torch.empty((N, sum(chans), HW), device="cuda")
    src = (ctypes.c_void_p * K)(*[t.data_ptr() for t in xd])
    ch = (ctypes.c_int64 * K)(*chans)
    ok(gn, L.soar_concat_channels_forward(src, ch, K, P(out), N, HW, None))
    want = np.concatenate(xs, axis=1)
    np.testing.assert_array_equal(host(torch, out), want)
    g = r.normal(size=want.shape).astype(F32)
    gd = dev(torch, g)
    pre = [r.normal(size=(N, c, HW)).astype(F32) for c in chans]
    gi = [torch.full((N, c, HW), float("nan"), device="cuda") for c in chans]
    gi[1] = dev(torch, pre[1])  # added into
    gi[3] = dev(torch, pre[3])  # skipped (NULL), must stay as it was
    ptrs = (ctypes.c_void_p * K)(gi[0].data_ptr(), gi[1].data_ptr(), gi[2].data_ptr(), None)
    flags = (ctypes.c_uint * K)(0, gn.GN_ACCUMULATE_DX, 0, 0)
    ok(gn, L.soar_concat_channels_backward(P(gd), ptrs, ch, flags, K, N, HW, None))
    offs = np.cumsum([0] + chans)
    np.testing.assert_array_equal(host(torch, gi[0]), g[:, offs[0]:offs[1]])
    np.testing.assert_array_equal(host(torch, gi[1]), pre[1] + g[:, offs[1]:offs[2]])
    np.testing.assert_array_equal(host(torch, gi[2]), g[:, offs[2]:offs[3]])
    np.testing.assert_array_equal(host(torch, gi[3]), pre[3])


# ---- write-mode backward entry points ----------------------------------------------
def test_backward_write_mode(env):
    """Every _ex backward with flags 0 overwrites its outputs (prefilled
    with NaN here) with exactly what the adding entry point adds to zeros,
    and with SOAR_GN_ACCUMULATE_DX equals the adding entry point."""
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(11)
    ACC = gn.GN_ACCUMULATE_DX
    C, H, W = 6, 10, 12
    n = C * H * W
    gy = dev(torch, r.normal(size=n))
    a = dev(torch, r.normal(size=n))
    b = dev(torch, r.normal(size=n))
    g = dev(torch, r.uniform(size=n))
    bc = dev(torch, r.normal(size=C))
    y01 = dev(torch, (r.uniform(size=n) < 0.4).astype(F32))
    go_up = dev(torch, r.normal(size=C * (2 * H) * (2 * W)))
    go_pool = dev(torch, r.normal(size=C))
    cases = {
        "sigmoid": ([n], lambda o, f: L.soar_sigmoid_backward_ex(P(gy), P(g), P(o[0]), n, f,
                                                                  None),
                    lambda o: L.soar_sigmoid_backward(P(gy), P(g), P(o[0]), n, None)),
        "mul_broadcast": ([n, C],
                          lambda o, f: L.soar_mul_broadcast_backward_ex(
                              P(gy), P(a), P(bc), P(o[0]), P(o[1]), C, H * W, f, None),
                          lambda o: L.soar_mul_broadcast_backward(
                              P(gy), P(a), P(bc), P(o[0]), P(o[1]), C, H * W, None)),
        "convex": ([n, n, n],
                   lambda o, f: L.soar_convex_combination_backward_ex(
                       P(gy), P(g), P(a), P(b), P(o[0]), P(o[1]), P(o[2]), n, f, None),
                   lambda o: L.soar_convex_combination_backward(
                       P(gy), P(g), P(a), P(b), P(o[0]), P(o[1]), P(o[2]), n, None)),
        "avg_pool": ([n], lambda o, f: L.soar_global_avg_pool_backward_ex(
                         P(go_pool), P(o[0]), C, H * W, f, None),
                     lambda o: L.soar_global_avg_pool_backward(P(go_pool), P(o[0]), C, H * W,
                                                               None)),
        "upsample_2x": ([n], lambda o, f: L.soar_upsample_bilinear_backward_ex(
                            P(go_up), P(o[0]), C, H, W, 2 * H, 2 * W, f, None),
                        lambda o: L.soar_upsample_bilinear_backward(
                            P(go_up), P(o[0]), C, H, W, 2 * H, 2 * W, None)),
        "upsample_tiled": ([n], lambda o, f: L.soar_upsample_bilinear_backward_ex(
                               P(go_up), P(o[0]), C, H, W, 2 * H - 1, 2 * W - 3, f, None),
                           lambda o: L.soar_upsample_bilinear_backward(
                               P(go_up), P(o[0]), C, H, W, 2 * H - 1, 2 * W - 3, None)),
        "upsample_wide": ([C * 2 * 2], lambda o, f: L.soar_upsample_bilinear_backward_ex(
                              P(go_up), P(o[0]), C, 2, 2, 2 * H, 2 * W, f, None),
                          lambda o: L.soar_upsample_bilinear_backward(
                              P(go_up), P(o[0]), C, 2, 2, 2 * H, 2 * W, None)),
        # 24 channels of 5 x 6 <-> 6 channels of 10 x 12
        "pixel_shuffle": ([n], lambda o, f: L.soar_pixel_shuffle_backward_ex(
                              P(gy), P(o[0]), 24, H // 2, W // 2, 2, f, None),
                          lambda o: L.soar_pixel_shuffle_backward(P(gy), P(o[0]), 24, H // 2,
                                                                  W // 2, 2, None)),
        "dice_bce": ([n], lambda o, f: L.soar_dice_bce_loss_backward_ex(
                         P(a), P(y01), P(o[0]), 1.0, 1.0, 0.5, 0.5, 3.0, 1.0, 30.0, 200.0,
                         250.0, n, f, None),
                     lambda o: L.soar_dice_bce_loss_backward(
                         P(a), P(y01), P(o[0]), 1.0, 1.0, 0.5, 0.5, 3.0, 1.0, 30.0, 200.0,
                         250.0, n, None)),
    }
    for name, (sizes, ex, plain) in cases.items():
        fresh = [torch.full((k,), float("nan"), device="cuda") for k in sizes]
        ok(gn, ex(fresh, 0))
        zeros = [torch.zeros(k, device="cuda") for k in sizes]
        ok(gn, plain(zeros))
        for f_, z_ in zip(fresh, zeros):
            np.testing.assert_array_equal(host(torch, f_), host(torch, z_), err_msg=name)
        pre = [dev(torch, r.normal(size=k)) for k in sizes]
        pre2 = [t.clone() for t in pre]
        ok(gn, ex(pre, ACC))
        ok(gn, plain(pre2))
        for p_, q_ in zip(pre, pre2):
            np.testing.assert_array_equal(host(torch, p_), host(torch, q_), err_msg=name)
        assert ex(fresh, 2) == gn.SOAR_EINVAL, name


# ---- AdamW and multi-tensor ---------------------------------------------------------
def test_adamw_and_multi_tensor(env):
    gn, torch = env
    L = gn.lib()
    r = np.random.default_rng(9)
    sizes = [1, 3, 4095, 4096, 4097, 70000, 16, 0, 300000] + [int(s) for s in r.integers(1, 5000, 200)]
    th = [r.normal(size=s).astype(F32) for s in sizes]
    g = [(r.normal(size=s) * 10.0 ** r.uniform(-4, 1)).astype(F32) for s in sizes]
    td = [dev(torch, a) if a.size else torch.empty(1, device="cuda") for a in th]
    gd = [dev(torch, a) if a.size else torch.empty(1, device="cuda") for a in g]
    md = [torch.zeros(max(s, 1), device="cuda") for s in sizes]
    vd = [torch.zeros(max(s, 1), device="cuda") for s in sizes]
    n = len(sizes)
    arr = lambda ts: (ctypes.c_void_p * n)(*[t.data_ptr() for t in ts])  # noqa: E731
    numel = (ctypes.c_int64 * n)(*sizes)
    m_ref = [np.zeros(s, F32) for s in sizes]
    v_ref = [np.zeros(s, F32) for s in sizes]
    for step in (1, 2, 3):
        lr = 1e-3 / step
        b1c = F32(1) - np.power(F32(0.9), F32(step), dtype=F32)
        b2c = F32(1) - np.power(F32(0.999), F32(step), dtype=F32)
        ok(gn, L.soar_adamw_step_multi_tensor(arr(td), arr(gd), arr(md), arr(vd), numel, n, lr, 0.9,
                                              0.999, 1e-8, 1e-2, F32(F32(lr) / b1c),
                                              np.sqrt(b2c, dtype=F32), None))
        for i in range(n):
            th[i], m_ref[i], v_ref[i] = smr.adamw_step(th[i], g[i], m_ref[i], v_ref[i], step, lr=lr)
        got = [host(torch, t)[:s] for t, s in zip(td, sizes)]
        for i in range(n):
            np.testing.assert_array_equal(got[i], th[i], err_msg=f"step {step} tensor {i}")
    # device-table forms: norm, scale, fill
    tab = torch.tensor([t.data_ptr() for t in gd], dtype=torch.int64, device="cuda")
    nm = torch.tensor(sizes, dtype=torch.int64, device="cuda")
    out = torch.zeros(1, dtype=torch.float64, device="cuda")
    wsb = L.soar_multi_tensor_norm_workspace_bytes()
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    ok(gn, L.soar_multi_tensor_norm_sq_device(P(tab), P(nm), n, P(out), P(ws), wsb, None))
    want = sum(float(np.dot(a.astype(np.float64), a)) for a in g)
    assert abs(float(host(torch, out)[0]) - want) <= 1e-12 * want
    ok(gn, L.soar_multi_tensor_scale_device(P(tab), P(nm), n, F32(0.5), None))
    for t, a in zip(gd, g):
        np.testing.assert_array_equal(host(torch, t)[:a.size], a * F32(0.5))
    ok(gn, L.soar_multi_tensor_fill_device(P(tab), P(nm), n, 0.0, None))
    assert all(not np.any(host(torch, t)[:s]) for t, s in zip(gd, sizes))
    # the single-tensor form
    x = r.normal(size=1000).astype(F32)
    gg = r.normal(size=1000).astype(F32)
    xd, ggd = dev(torch, x), dev(torch, gg)
    m1, v1 = torch.zeros(1000, device="cuda"), torch.zeros(1000, device="cuda")
    ok(gn, L.soar_adamw_step(P(xd), P(ggd), P(m1), P(v1), 1e-3, 0.9, 0.999, 1e-8, 1e-2,
                             F32(F32(1e-3) / (F32(1) - F32(0.9))),
                             np.sqrt(F32(1) - F32(0.999), dtype=F32), 1000, None))
    t1, _, _ = smr.adamw_step(x, gg, np.zeros(1000, F32), np.zeros(1000, F32), 1)
    np.testing.assert_array_equal(host(torch, xd), t1)
    # a table over the limit is refused before any launch
    assert L.soar_multi_tensor_fill_device(P(tab), P(nm), 4096, 0.0, None) == gn.SOAR_EINVAL


@pytest.mark.parametrize("max_norm,zero", [(2.0, True), (1e9, True), (2.0, False)])
def test_fused_clip_adamw_tail(env, max_norm, zero):
    """soar_multi_tensor_norm_sq_partials_device + soar_adamw_clip_multi_tensor_
    device give bit for bit what norm_sq_device, clip_device, adamw_multi_
    tensor_device_scalars and (with SOAR_ADAMW_ZERO_GRAD) fill_device(0)
    give: parameters, moments, the squared norm and the gradients after
    the step; clipping on (max_norm 2) and off (1e9)."""
    gn, torch = env
    L = gn.lib()
    print(f"case: fused clip + AdamW max_norm={max_norm} zero={zero}", flush=True)
    r = np.random.default_rng(21)
    sizes = [5, 4096, 70001, 3, 12000]
    n = len(sizes)
    th = [r.normal(size=s).astype(F32) for s in sizes]
    gr = [(r.normal(size=s) * 0.05).astype(F32) for s in sizes]
    mo = [(r.normal(size=s) * 1e-3).astype(F32) for s in sizes]
    ve = [np.abs(r.normal(size=s) * 1e-4).astype(F32) for s in sizes]
    wsb = L.soar_multi_tensor_norm_workspace_bytes()
    sc = torch.tensor([1e-3, 1e-3 / 0.1, np.sqrt(1 - 0.999)], dtype=torch.float32, device="cuda")
    runs = []
    for fused in (False, True):
        P_, G_, M_, V_ = ([dev(torch, a) for a in arrs] for arrs in (th, gr, mo, ve))
        tab = lambda ts: torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64,  # noqa: E731
                                      device="cuda")
        tp, tg, tm, tv = tab(P_), tab(G_), tab(M_), tab(V_)
        nm = torch.tensor(sizes, dtype=torch.int64, device="cuda")
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        norm = torch.zeros(1, dtype=torch.float64, device="cuda")
        if fused:
            ok(gn, L.soar_multi_tensor_norm_sq_partials_device(P(tg), P(nm), n, P(ws), wsb, None))
            ok(gn, L.soar_adamw_clip_multi_tensor_device(
                P(tp), P(tg), P(tm), P(tv), P(nm), n, P(sc), 0.9, 0.999, 1e-8, 1e-2, P(ws), wsb,
                max_norm, P(norm), gn.ADAMW_ZERO_GRAD if zero else 0, None))
        else:
            ok(gn, L.soar_multi_tensor_norm_sq_device(P(tg), P(nm), n, P(norm), P(ws), wsb, None))
            ok(gn, L.soar_multi_tensor_clip_device(P(tg), P(nm), n, P(norm), max_norm, None))
            ok(gn, L.soar_adamw_multi_tensor_device_scalars(P(tp), P(tg), P(tm), P(tv), P(nm), n,
                                                            P(sc), 0.9, 0.999, 1e-8, 1e-2,
                                                            None))
            if zero:
                ok(gn, L.soar_multi_tensor_fill_device(P(tg), P(nm), n, 0.0, None))
        runs.append([host(torch, t) for t in P_ + G_ + M_ + V_ + [norm]])
    for k, (a, b) in enumerate(zip(*runs)):
        np.testing.assert_array_equal(a, b, err_msg=f"tensor {k}")
    want = sum(float(np.dot(a.astype(np.float64), a)) for a in gr)
    assert abs(float(runs[1][-1][0]) - want) <= 1e-12 * want
    clipped = np.sqrt(want) > max_norm
    if zero:
        assert all(not np.any(runs[1][n + i]) for i in range(n))
    elif clipped:
        assert not np.array_equal(runs[1][n], gr[0])
    assert L.soar_adamw_clip_multi_tensor_device(None, None, None, None, None, 0, None, 0.9,
                                                 0.999, 1e-8, 0.0, None, 0, 1.0, None, 2,
                                                 None) == gn.SOAR_EINVAL
