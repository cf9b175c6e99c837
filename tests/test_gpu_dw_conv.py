"""Parity of the depthwise convolution (forward and backward, through the
C-ABI of libsoar_gn.so) against the float64 oracle.

Bars (written here):
  y  : |y - y64|   <= (K*K + 2) * 2^-24 * (|w| (*) |x| + |b|)
  dx : |dx - dx64| <= (K*K + 2) * 2^-24 * (|w| scattered |dy|)
  dw, db : |d - d64| <= (P + 2) * 2^-24 * (sum of |terms|), P the number of
           summed products (the fp32 bound of a P-term sum, any order)
"""
import numpy as np
import pytest

from test_gpu_parity import dev, host

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


def autopad(K, d):
    k = d * (K - 1) + 1 if d > 1 else K
    return k // 2


CASES = [
    # (N, C, H, W, K, stride, dil): the model's configurations, tile edges
    (1, 4, 70, 130, 3, 1, 1),
    (2, 3, 67, 131, 3, 2, 1),     # Down.dw, odd sizes
    (1, 2, 64, 128, 5, 1, 1),     # exact tiles
    (1, 3, 45, 200, 7, 1, 1),     # LKR k=7
    (1, 2, 40, 70, 3, 1, 2),
    (1, 2, 50, 66, 3, 1, 3),      # Ctx
    (1, 2, 33, 90, 3, 1, 5),
    (1, 2, 20, 21, 4, 2, 2),      # generic kernels (even K, stride 2, dilation 2)
    (1, 2, 13, 17, 5, 3, 1),      # generic, stride 3
    (2, 3, 5, 7, 7, 1, 1),        # image smaller than the kernel
    # one sample, one output tile per plane: the weight-gradient blocks add
    # their sums into dw / db directly (no finish kernel)
    (1, 4, 32, 64, 3, 1, 1),
    (1, 3, 17, 30, 7, 1, 1),
    (1, 5, 24, 40, 3, 2, 1),
    (1, 2, 10, 12, 3, 1, 3),
    (1, 2, 30, 60, 5, 1, 1),
]


def inputs(seed, N, C, H, W, K):
    r = np.random.default_rng(seed)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = r.uniform(-1, 1, (C, K, K)).astype(np.float32) / K
    b = r.uniform(-0.5, 0.5, C).astype(np.float32)
    return x, w, b


def check(got, truth, bound, name):
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - np.asarray(truth).reshape(-1))
    bd = np.asarray(bound).reshape(-1) + 1e-30
    i = int(np.argmax(err / bd))
    assert err[i] <= bd[i], f"{name} err {err[i]:.3e} > bound {bd[i]:.3e} at {i}"


@pytest.mark.parametrize("N,C,H,W,K,s,d", CASES)
def test_dw_forward_matches_oracle(gpu, oracle, N, C, H, W, K, s, d):
    print(f"dw fwd N={N} C={C} {H}x{W} K={K} s={s} d={d}", flush=True)
    pad = autopad(K, d)
    x, w, b = inputs(H * W + K, N, C, H, W, K)
    y = gpu.dw_conv_forward(dev(x), dev(w), dev(b), pad, s, d)
    t = oracle.dw_fwd_f64(x, w, b, N, C, H, W, K, pad, s, d)
    assert tuple(y.shape) == t.shape
    mag = oracle.dw_fwd_f64(np.abs(x), np.abs(w), np.abs(b), N, C, H, W, K, pad, s, d)
    check(host(y), t, (K * K + 2) * U32 * mag, "y")


@pytest.mark.parametrize("N,C,H,W,K,s,d", CASES)
def test_dw_backward_matches_oracle(gpu, oracle, N, C, H, W, K, s, d):
    print(f"dw bwd N={N} C={C} {H}x{W} K={K} s={s} d={d}", flush=True)
    pad = autopad(K, d)
    x, w, _ = inputs(H * W + K + 1, N, C, H, W, K)
    Ho, Wo = oracle.dw_out_size(H, K, pad, s, d), oracle.dw_out_size(W, K, pad, s, d)
    dy = np.random.default_rng(K).standard_normal((N, C, Ho, Wo)).astype(np.float32)
    dx, dw, db = gpu.dw_conv_backward(dev(dy), dev(x), dev(w), pad, s, d)
    tx, tw, tb = oracle.dw_bwd_f64(dy, x, w, N, C, H, W, K, pad, s, d)
    ax, aw, _ = oracle.dw_bwd_f64(np.abs(dy), np.abs(x), np.abs(w), N, C, H, W, K, pad, s, d)
    check(host(dx), tx, (K * K + 2) * U32 * ax, "dx")
    P = N * Ho * Wo + 2
    check(host(dw), tw, P * U32 * aw, "dw")
    check(host(db), tb, P * U32 * np.abs(dy).sum(axis=(0, 2, 3)), "db")
    # small layers run dx and the weight gradient in one launch
    # (k_dw_bwd_small): the same bits as each alone
    dx1, _, _ = gpu.dw_conv_backward(dev(dy), dev(x), dev(w), pad, s, d, want_dw=False,
                                     want_db=False)
    _, dw1, db1 = gpu.dw_conv_backward(dev(dy), dev(x), dev(w), pad, s, d, want_dx=False)
    for a, b_, name in ((dx1, dx, "dx"), (dw1, dw, "dw"), (db1, db, "db")):
        assert np.array_equal(host(a), host(b_)), f"{name} alone vs together"


@pytest.mark.parametrize("H,W", [(40, 70), (20, 30)])  # partials + finish, direct
def test_dw_backward_accumulates_and_skips(gpu, oracle, H, W):
    N, C, K, s, d = 1, 3, 3, 1, 1
    pad = autopad(K, d)
    x, w, _ = inputs(3, N, C, H, W, K)
    dy = np.random.default_rng(4).standard_normal((N, C, H, W)).astype(np.float32)
    r = np.random.default_rng(5)
    dx0 = r.standard_normal((N, C, H, W)).astype(np.float32)
    dw0 = r.standard_normal((C, K, K)).astype(np.float32)
    db0 = r.standard_normal(C).astype(np.float32)
    dx, dw, db = gpu.dw_conv_backward(dev(dy), dev(x), dev(w), pad, s, d, dx=dev(dx0),
                                      dweight=dev(dw0), dbias=dev(db0), accumulate_dx=True)
    tx, tw, tb = oracle.dw_bwd_f64(dy, x, w, N, C, H, W, K, pad, s, d)
    ax, aw, _ = oracle.dw_bwd_f64(np.abs(dy), np.abs(x), np.abs(w), N, C, H, W, K, pad, s, d)
    check(host(dx), dx0 + tx, (K * K + 3) * U32 * (ax + np.abs(dx0)), "dx+=")
    P = N * H * W + 3
    check(host(dw), dw0 + tw, P * U32 * (aw + np.abs(dw0)), "dw+=")
    check(host(db), db0 + tb, P * U32 * (np.abs(dy).sum(axis=(0, 2, 3)) + np.abs(db0)), "db+=")
    dx2, dw2, db2 = gpu.dw_conv_backward(dev(dy), dev(x), dev(w), pad, s, d, want_dx=False,
                                         want_dw=False)
    assert dx2 is None and dw2 is None
    check(host(db2), tb, P * U32 * np.abs(dy).sum(axis=(0, 2, 3)), "db only")


def test_reference_signature_dw(gpu, oracle):
    """soar_conv2d_dw_forward / soar_conv2d_dw_backward (one sample; the
    backward accumulates) against the fp32 statement of the reference."""
    import ctypes
    import torch
    C, H, W, K, s, d = 4, 33, 65, 5, 1, 1
    pad = autopad(K, d)
    x, w, b = inputs(6, 1, C, H, W, K)
    Ho, Wo = oracle.dw_out_size(H, K, pad, s, d), oracle.dw_out_size(W, K, pad, s, d)
    xd, wd, bd = dev(x[0]), dev(w), dev(b)
    y = torch.empty((C, Ho, Wo), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    L = gpu.lib()
    gpu.check(L.soar_conv2d_dw_forward(P(xd), P(wd), P(bd), P(y), C, H, W, Ho, Wo, K, pad, s, d,
                                       None))
    torch.cuda.synchronize()
    ref = oracle.ref_dw_fwd_f32(x[0], w, b, C, H, W, K, pad, s, d)
    mag = oracle.dw_fwd_f64(np.abs(x), np.abs(w), np.abs(b), 1, C, H, W, K, pad, s, d)[0]
    check(host(y), ref, 2 * (K * K + 2) * U32 * mag, "ref y")
    dy = np.random.default_rng(7).standard_normal((C, Ho, Wo)).astype(np.float32)
    dyd = dev(dy)
    gi = torch.zeros((C, H, W), device="cuda")
    gw = torch.zeros((C, K, K), device="cuda")
    gb = torch.zeros(C, device="cuda")
    gpu.check(L.soar_conv2d_dw_backward(P(dyd), P(xd), P(wd), P(gi), P(gw), P(gb), C, H, W, Ho,
                                        Wo, K, pad, s, d, None))
    torch.cuda.synchronize()
    ri, rw, rb = oracle.ref_dw_bwd_f32(dy, x[0], w, C, H, W, K, pad, s, d)
    ax, aw, _ = oracle.dw_bwd_f64(np.abs(dy)[None], np.abs(x), np.abs(w), 1, C, H, W, K, pad, s,
                                  d)
    Pn = Ho * Wo + 2
    check(host(gi), ri, 2 * (K * K + 2) * U32 * ax, "ref dx")
    check(host(gw), rw, 2 * Pn * U32 * aw, "ref dw")
    check(host(gb), rb, 2 * Pn * U32 * np.abs(dy).sum(axis=(1, 2)), "ref db")


def test_dw_full_size_lkr(gpu):
    """LKR.dw (k7, stride 1) at 64 x 2048 x 2048: the forward and dx on 64
    random 7x7 windows against float64, and the adjoint identities
    <y - b, dy> = <x, dx> = <w, dw> at full size."""
    import torch
    C, H, K = 64, 2048, 7
    pad = autopad(K, 1)
    print("dw full size 64x2048^2 k7", flush=True)
    x = torch.empty((1, C, H, H), device="cuda")
    dy = torch.empty((1, C, H, H), device="cuda")
    gpu.synth_normal(x, 91, 1)
    gpu.synth_normal(dy, 91, 4)
    r = np.random.default_rng(11)
    w = dev((r.uniform(-1, 1, (C, K, K)) / K).astype(np.float32))
    y = gpu.dw_conv_forward(x, w, None, pad)
    dx, dw, db = gpu.dw_conv_backward(dy, x, w, pad)
    torch.cuda.synchronize()
    ydy = torch.dot(y.reshape(-1).double(), dy.reshape(-1).double()).item()
    xdx = torch.dot(x.reshape(-1).double(), dx.reshape(-1).double()).item()
    wdw = torch.dot(w.reshape(-1).double(), dw.reshape(-1).double()).item()
    scale = torch.dot(y.reshape(-1).double().abs(), dy.reshape(-1).double().abs()).item()
    assert abs(xdx - ydy) <= 1e-5 * scale, (xdx, ydy, scale)
    assert abs(wdw - ydy) <= 1e-5 * scale, (wdw, ydy, scale)
    wh = host(w).astype(np.float64)
    for i in range(64):
        c = int(r.integers(C))
        yo, xo = (int(v) for v in r.integers(0, H, 2))
        acc = 0.0
        mag = 0.0
        for ky in range(K):
            for kx in range(K):
                yi, xi = yo - pad + ky, xo - pad + kx
                if 0 <= yi < H and 0 <= xi < H:
                    v = float(x[0, c, yi, xi]) * wh[c, ky, kx]
                    acc += v
                    mag += abs(v)
        assert abs(float(y[0, c, yo, xo]) - acc) <= (K * K + 2) * U32 * mag + 1e-30
    del x, dy, y, dx


@pytest.mark.parametrize("K,S,D,H", [(7, 1, 1, 300), (3, 2, 1, 257), (3, 1, 5, 130)])
def test_dw_paths_are_deterministic(gpu, K, S, D, H):
    """Multi-tile depthwise kernels and the weight-gradient finish sum in a
    fixed order: two runs are bitwise identical."""
    import torch
    print(f"dw determinism K={K} S={S} D={D} H={H}", flush=True)
    C = 24
    pad = (D * (K - 1) + 1) // 2 if D > 1 else K // 2
    r = np.random.default_rng(K * 100 + H)
    x = torch.from_numpy(r.standard_normal((2, C, H, H)).astype(np.float32)).cuda()
    w = torch.from_numpy((r.standard_normal((C, K, K)) / K).astype(np.float32)).cuda()
    b = torch.from_numpy(r.standard_normal(C).astype(np.float32)).cuda()
    Ho = gpu.conv_out_size(H, K, pad, S, D)
    dy = torch.from_numpy(r.standard_normal((2, C, Ho, Ho)).astype(np.float32)).cuda()
    runs = []
    for _ in range(2):
        y = gpu.dw_conv_forward(x, w, b, pad, S, D)
        dx, dw, db = gpu.dw_conv_backward(dy, x, w, pad, S, D)
        runs.append([t.cpu().numpy() for t in (y, dx, dw, db)])
    for a, c in zip(*runs):
        assert np.array_equal(a, c)
