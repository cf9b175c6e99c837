"""Pins of the oracle's pointwise convolution (oracle/soar_oracle.c) - CPU.

orc_conv1x1_fwd_f64 is checked against numpy's float64 matrix product (an
independent implementation: BLAS), closed forms chosen so a transposed
weight, a wrong plane stride or a dropped bias fails, and linearity.
ref_conv1x1_fwd_f32 (the reference's per-output loop,
src/cuda/ops/convolution_kernels.cu:10-31) is checked against the float64
truth within the fp32 bound of a K-term dot product.
"""
import numpy as np
import pytest

U32 = 2.0 ** -24  # unit roundoff of float32


def rand(shape, seed, lo=-1.0, hi=1.0):
    r = np.random.default_rng(seed)
    return r.uniform(lo, hi, size=shape).astype(np.float32)


@pytest.mark.parametrize("N,C_in,C_out,HW", [(1, 3, 5, 7), (2, 16, 24, 33), (1, 64, 64, 257)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv_f64_matches_numpy(oracle, N, C_in, C_out, HW, with_bias):
    x = rand((N, C_in, HW), 1)
    w = rand((C_out, C_in), 2)
    b = rand((C_out,), 3) if with_bias else None
    y = oracle.conv1x1_fwd_f64(x, w, b, N, C_in, C_out, HW).reshape(N, C_out, HW)
    ref = np.einsum("oc,ncp->nop", w.astype(np.float64), x.astype(np.float64))
    if with_bias:
        ref += b.astype(np.float64)[None, :, None]
    np.testing.assert_allclose(y, ref, rtol=1e-13, atol=1e-13)


def test_conv_f64_closed_forms(oracle):
    N, C, HW = 2, 6, 11
    x = rand((N, C, HW), 4)
    # identity weights reproduce the input exactly
    y = oracle.conv1x1_fwd_f64(x, np.eye(C, dtype=np.float32), None, N, C, C, HW)
    np.testing.assert_array_equal(y.reshape(N, C, HW), x.astype(np.float64))
    # a one-hot row selects one input channel (catches a transposed weight)
    w = np.zeros((3, C), dtype=np.float32)
    w[0, 4] = 1.0
    w[1, 1] = 2.0
    w[2, 5] = -1.0
    y = oracle.conv1x1_fwd_f64(x, w, None, N, C, 3, HW).reshape(N, 3, HW)
    np.testing.assert_array_equal(y[:, 0], x[:, 4])
    np.testing.assert_array_equal(y[:, 1], 2.0 * x[:, 1].astype(np.float64))
    np.testing.assert_array_equal(y[:, 2], -x[:, 5].astype(np.float64))
    # zero weights give the bias broadcast over pixels and samples
    b = np.array([0.5, -2.0, 3.25], dtype=np.float32)
    y = oracle.conv1x1_fwd_f64(x, np.zeros((3, C), np.float32), b, N, C, 3, HW)
    np.testing.assert_array_equal(y.reshape(N, 3, HW), np.broadcast_to(b[None, :, None],
                                                                       (N, 3, HW)))


def test_conv_f64_linearity(oracle):
    N, C_in, C_out, HW = 1, 8, 5, 64
    x1, x2 = rand((N, C_in, HW), 5), rand((N, C_in, HW), 6)
    w = rand((C_out, C_in), 7)
    y1 = oracle.conv1x1_fwd_f64(x1, w, None, N, C_in, C_out, HW)
    y2 = oracle.conv1x1_fwd_f64(x2, w, None, N, C_in, C_out, HW)
    y12 = oracle.conv1x1_fwd_f64(x1.astype(np.float64) + x2, w, None, N, C_in, C_out, HW)
    # x1 + x2 is rounded to fp32 by the wrapper; compare against that input
    xs = (x1.astype(np.float64) + x2).astype(np.float32)
    ys = oracle.conv1x1_fwd_f64(xs, w, None, N, C_in, C_out, HW)
    np.testing.assert_array_equal(y12, ys)
    bound = C_in * U32 * (np.abs(w).astype(np.float64) @ (np.abs(x1) + np.abs(x2))[0])
    assert np.all(np.abs(ys - (y1 + y2)) <= bound.reshape(-1) + 1e-12)


@pytest.mark.parametrize("C_in,C_out,HW", [(1, 1, 5), (7, 3, 50), (64, 64, 512)])
def test_reference_conv_port_tracks_truth(oracle, C_in, C_out, HW):
    x = rand((C_in, HW), 8)
    w = rand((C_out, C_in), 9)
    b = rand((C_out,), 10)
    y = oracle.ref_conv1x1_fwd_f32(x, w, b, C_in, C_out, HW).astype(np.float64)
    t = oracle.conv1x1_fwd_f64(x, w, b, 1, C_in, C_out, HW)
    mag = np.abs(w).astype(np.float64) @ np.abs(x).astype(np.float64) + np.abs(b)[:, None]
    assert np.all(np.abs(y - t) <= (C_in + 1) * U32 * mag.reshape(-1) + 1e-30)


@pytest.mark.parametrize("N,C_in,C_out,HW", [(1, 3, 5, 7), (2, 16, 24, 33)])
def test_conv_bwd_f64_matches_numpy(oracle, N, C_in, C_out, HW):
    dz = rand((N, C_out, HW), 11)
    x = rand((N, C_in, HW), 12)
    w = rand((C_out, C_in), 13)
    dx, dw, db = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    d64, x64, w64 = (a.astype(np.float64) for a in (dz, x, w))
    np.testing.assert_allclose(dx.reshape(N, C_in, HW), np.einsum("oc,nop->ncp", w64, d64),
                               rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(dw.reshape(C_out, C_in), np.einsum("nop,ncp->oc", d64, x64),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, d64.sum(axis=(0, 2)), rtol=1e-13, atol=1e-13)


def test_conv_bwd_f64_is_the_adjoint(oracle):
    """<conv(x), dz> = <x, conv^T(dz)> and d<conv(x), dz>/dW = dW: the
    backward is the exact adjoint of the forward (catches a transposed W)."""
    N, C_in, C_out, HW = 2, 5, 7, 19
    x = rand((N, C_in, HW), 14)
    w = rand((C_out, C_in), 15)
    b = rand((C_out,), 16)
    dz = rand((N, C_out, HW), 17)
    z = oracle.conv1x1_fwd_f64(x, w, b, N, C_in, C_out, HW)
    dx, dw, db = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    lhs = float(np.dot(z, dz.reshape(-1).astype(np.float64)))
    rhs = float(np.dot(x.reshape(-1).astype(np.float64), dx)) + float(
        np.dot(b.astype(np.float64), db))
    assert abs(lhs - rhs) <= 1e-10 * (1 + abs(lhs))
    # <z, dz> is linear in W with gradient dw
    h = 1e-3
    w2 = w.copy()
    w2[3, 2] += h
    z2 = oracle.conv1x1_fwd_f64(x, w2, b, N, C_in, C_out, HW)
    fd = (float(np.dot(z2, dz.reshape(-1).astype(np.float64))) - lhs) / (float(w2[3, 2]) -
                                                                         float(w[3, 2]))
    assert abs(fd - dw[3 * C_in + 2]) <= 1e-6 * (1 + abs(fd))


@pytest.mark.parametrize("C_in,C_out,HW", [(1, 1, 5), (7, 3, 50), (32, 16, 300)])
def test_reference_conv_bwd_port_tracks_truth(oracle, C_in, C_out, HW):
    go = rand((C_out, HW), 18)
    x = rand((C_in, HW), 19)
    w = rand((C_out, C_in), 20)
    gi0 = rand((C_in * HW,), 21)  # accumulates into what is there
    gi, gw, gb = oracle.ref_conv1x1_bwd_f32(go, x, w, C_in, C_out, HW, grad_in=gi0.copy())
    dx, dw, db = oracle.conv1x1_bwd_f64(go, x, w, 1, C_in, C_out, HW)
    magx = np.abs(w).astype(np.float64).T @ np.abs(go).astype(np.float64)
    assert np.all(np.abs(gi - (gi0 + dx)) <= (C_out + 2) * U32 * (magx.reshape(-1) + np.abs(gi0)))
    magw = np.abs(go).astype(np.float64) @ np.abs(x).astype(np.float64).T
    assert np.all(np.abs(gw - dw) <= (HW + 1) * U32 * magw.reshape(-1) + 1e-30)
    assert np.all(np.abs(gb - db) <= (HW + 1) * U32 * np.abs(go).sum(axis=1) + 1e-30)
