"""Pins of the oracle's depthwise convolution (oracle/soar_oracle.c) - CPU.

orc_dw_fwd_f64 / orc_dw_bwd_f64 are checked against an independent numpy
formulation (zero-padded input, one strided slice per tap), closed forms
(a centred delta kernel is the identity, an off-centre delta a shift) and
the adjoint identity <conv(x), dy> = <x, dx> + <w, dw> + <b, db>, which
fails for a flipped kernel or a misplaced tap in the backward.  The fp32
statements of the reference kernels are checked against the float64 truth
within the fp32 bound of a K*K-term (or pixel-count-term) sum.
"""
import numpy as np
import pytest

U32 = 2.0 ** -24

CASES = [
    # (N, C, H, W, K, stride, dil) with the reference's autopad
    (1, 3, 9, 11, 3, 1, 1),
    (2, 2, 10, 7, 3, 2, 1),    # Down.dw
    (1, 2, 12, 13, 5, 1, 1),   # LKR k=5
    (1, 1, 15, 16, 7, 1, 1),   # LKR k=7
    (1, 2, 17, 14, 3, 1, 3),   # Ctx dilation 3
    (1, 1, 9, 9, 3, 1, 5),     # dilation wider than half the image
    (1, 2, 8, 9, 4, 2, 2),     # even kernel, stride 2, dilation 2
]


def autopad(K, d):
    """layers.hpp:16-19: pad = (d*(K-1)+1) // 2 for p < 0."""
    k = d * (K - 1) + 1 if d > 1 else K
    return k // 2


def rand(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, size=shape).astype(np.float32)


def np_dw_fwd(x, w, b, K, pad, s, d):
    N, C, H, W = x.shape
    Ho = (H + 2 * pad - (d * (K - 1) + 1)) // s + 1
    Wo = (W + 2 * pad - (d * (K - 1) + 1)) // s + 1
    xp = np.zeros((N, C, H + 2 * pad + s * Ho + d * K, W + 2 * pad + s * Wo + d * K))
    xp[:, :, pad:pad + H, pad:pad + W] = x
    y = np.zeros((N, C, Ho, Wo)) + (0 if b is None else b.astype(np.float64)[None, :, None, None])
    for ky in range(K):
        for kx in range(K):
            sl = xp[:, :, ky * d:ky * d + s * Ho:s, kx * d:kx * d + s * Wo:s]
            y += sl * w[:, ky, kx].astype(np.float64)[None, :, None, None]
    return y


@pytest.mark.parametrize("N,C,H,W,K,s,d", CASES)
def test_dw_fwd_matches_numpy(oracle, N, C, H, W, K, s, d):
    pad = autopad(K, d)
    x, w, b = rand((N, C, H, W), 1), rand((C, K, K), 2), rand((C,), 3)
    y = oracle.dw_fwd_f64(x, w, b, N, C, H, W, K, pad, s, d)
    np.testing.assert_allclose(y, np_dw_fwd(x, w, b, K, pad, s, d), rtol=1e-13, atol=1e-13)


def test_dw_fwd_closed_forms(oracle):
    N, C, H, W, K = 1, 2, 6, 7, 3
    x = rand((N, C, H, W), 4)
    w = np.zeros((C, K, K), np.float32)
    w[:, 1, 1] = 1.0  # centred delta with pad 1: identity
    y = oracle.dw_fwd_f64(x, w, None, N, C, H, W, K, 1, 1, 1)
    np.testing.assert_array_equal(y, x.astype(np.float64))
    w[:] = 0
    w[:, 0, 2] = 1.0  # tap (ky=0, kx=2): y[yo][xo] = x[yo-1][xo+1]
    y = oracle.dw_fwd_f64(x, w, None, N, C, H, W, K, 1, 1, 1)
    ref = np.zeros_like(y)
    ref[:, :, 1:, :-1] = x[:, :, :-1, 1:]
    np.testing.assert_array_equal(y, ref)
    # channel c only sees weight c (catches a channel mix-up)
    w = np.zeros((C, K, K), np.float32)
    w[1, 1, 1] = 2.0
    y = oracle.dw_fwd_f64(x, w, None, N, C, H, W, K, 1, 1, 1)
    np.testing.assert_array_equal(y[:, 0], 0.0)
    np.testing.assert_array_equal(y[:, 1], 2.0 * x[:, 1].astype(np.float64))


@pytest.mark.parametrize("N,C,H,W,K,s,d", CASES)
def test_dw_bwd_is_the_adjoint(oracle, N, C, H, W, K, s, d):
    pad = autopad(K, d)
    x, w, b = rand((N, C, H, W), 5), rand((C, K, K), 6), rand((C,), 7)
    y = oracle.dw_fwd_f64(x, w, b, N, C, H, W, K, pad, s, d)
    dy = rand(y.shape, 8)
    dx, dw, db = oracle.dw_bwd_f64(dy, x, w, N, C, H, W, K, pad, s, d)
    lhs = float(np.sum(y * dy.astype(np.float64)))
    # <y, dy> = <W*x, dy> + <b, sum dy>; W*x is linear in both x and w
    lin_x = float(np.sum(x.astype(np.float64) * dx))
    lin_w = float(np.sum(w.astype(np.float64) * dw))
    cb = float(np.dot(b.astype(np.float64), db))
    assert abs(lhs - (lin_x + cb)) <= 1e-11 * (1 + abs(lhs))
    assert abs(lhs - (lin_w + cb)) <= 1e-11 * (1 + abs(lhs))
    np.testing.assert_allclose(db, dy.astype(np.float64).sum(axis=(0, 2, 3)), rtol=1e-13)
    # dw against a finite difference of <y, dy> (exact: y is linear in w)
    c, ky, kx = C - 1, K // 2, K - 1
    w2 = w.copy()
    w2[c, ky, kx] += 0.5
    y2 = oracle.dw_fwd_f64(x, w2, b, N, C, H, W, K, pad, s, d)
    step = float(w2[c, ky, kx]) - float(w[c, ky, kx])  # 0.5 after fp32 rounding
    fd = (float(np.sum(y2 * dy.astype(np.float64))) - lhs) / step
    assert abs(fd - dw[c, ky, kx]) <= 1e-9 * (1 + abs(fd))


@pytest.mark.parametrize("N,C,H,W,K,s,d", CASES)
def test_reference_dw_ports_track_truth(oracle, N, C, H, W, K, s, d):
    pad = autopad(K, d)
    x, w, b = rand((1, C, H, W), 9), rand((C, K, K), 10), rand((C,), 11)
    y = oracle.ref_dw_fwd_f32(x, w, b, C, H, W, K, pad, s, d).astype(np.float64)
    t = oracle.dw_fwd_f64(x, w, b, 1, C, H, W, K, pad, s, d)[0]
    mag = np_dw_fwd(np.abs(x), np.abs(w), np.abs(b), K, pad, s, d)[0]
    assert np.all(np.abs(y - t) <= (K * K + 1) * U32 * mag + 1e-30)
    dy = rand(t.shape, 12)
    gi0 = rand((C * H * W,), 13)
    gi, gw, gb = oracle.ref_dw_bwd_f32(dy, x, w, C, H, W, K, pad, s, d, grad_in=gi0.copy())
    dx, dw, db = oracle.dw_bwd_f64(dy[None], x, w, 1, C, H, W, K, pad, s, d)
    # |dx| bound: the same scatter with absolute values
    _, adw_x, _ = oracle.dw_bwd_f64(np.abs(dy)[None], np.abs(x), np.abs(w), 1, C, H, W, K, pad,
                                    s, d)
    adx, _, _ = oracle.dw_bwd_f64(np.abs(dy)[None], np.abs(x), np.abs(w), 1, C, H, W, K, pad, s,
                                  d)
    assert np.all(np.abs(gi.reshape(-1) - (gi0 + dx.reshape(-1))) <=
                  (K * K + 2) * U32 * (adx.reshape(-1) + np.abs(gi0)) + 1e-30)
    P = t.size // C + 1
    assert np.all(np.abs(gw - dw) <= P * U32 * adw_x + 1e-30)
    assert np.all(np.abs(gb - db) <= P * U32 * np.abs(dy).reshape(C, -1).sum(axis=1) + 1e-30)
