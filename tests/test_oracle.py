"""Pins of the CPU oracle (oracle/soar_oracle.c) - runs on the CPU.

Each check is chosen so a plausible slip in the oracle (a dropped term, a
wrong sign or index, a transposed operand) fails it:
  * torch float64 autograd fixtures (an independent implementation);
  * central finite differences of the float64 forward;
  * closed forms and invariants of the GroupNorm algebra;
  * the reference's own known-answer test input and tolerance
    (tests/test_operators.cpp:200-320 of pomagrenate/soar.cpp);
  * the published splitmix64 test vector.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

EPS32 = float(np.float32(1e-5))


def load_cases():
    z = np.load(os.path.join(GOLDEN, "gn_silu_f64.npz"))
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


Z, NAMES = load_cases()


def case(name):
    g = {k.split("/")[1]: Z[k] for k in Z.files if k.startswith(name + "/")}
    N, C, HW, G, silu, res, affine = (int(v) for v in g["shape"])
    return g, N, C, HW, G, bool(silu), bool(res), bool(affine)


# ---------------------------------------------------------------- generator

def test_splitmix64_published_vector(oracle):
    # splitmix64 seeded with 1234567 (Vigna's reference implementation).
    L = oracle.lib()
    assert L.orc_splitmix64_at(1234567, 0) == 6457827717110365317
    assert L.orc_splitmix64_at(1234567, 1) == 3203168211198807973


def test_normal_generator_moments(oracle):
    x = oracle.fill_normal(1 << 20, 7, 1, 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.var() - 1.0) < 5e-3
    # the two halves of each Box-Muller pair are uncorrelated
    assert abs(np.corrcoef(x[0::2], x[1::2])[0, 1]) < 5e-3
    u = oracle.fill_uniform(1 << 20, 7, 2, 0.5, 1.5).astype(np.float64)
    assert 0.5 <= u.min() and u.max() < 1.5
    assert abs(u.mean() - 1.0) < 2e-3


def test_stress_generator(oracle):
    n = 1 << 20
    x = oracle.fill_stress(n, 11, center=1e3, std=1e-2, p=1e-3, out_mean=0.0, out_std=50.0)
    outl = np.abs(x - 1e3) > 1.0
    assert 0.0008 < outl.mean() < 0.0012
    assert abs(np.median(x) - 1e3) < 1e-3


# ------------------------------------------------------------- float64 truth

@pytest.mark.parametrize("name", NAMES)
def test_truth_forward_matches_torch_f64(oracle, name):
    g, N, C, HW, G, silu, res, affine = case(name)
    gamma = g["gamma"] if affine else None
    beta = g["beta"] if affine else None
    y, mean, rstd = oracle.gn_silu_fwd_f64(g["x"], gamma, beta, N, C, HW, G, 1e-5, silu, res)
    np.testing.assert_allclose(mean, g["mean"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(rstd, g["rstd"], rtol=1e-10)
    np.testing.assert_allclose(y, g["y"].reshape(-1), rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("name", NAMES)
def test_truth_backward_matches_torch_f64(oracle, name):
    g, N, C, HW, G, silu, res, affine = case(name)
    gamma = g["gamma"] if affine else None
    beta = g["beta"] if affine else None
    _, mean, rstd = oracle.gn_silu_fwd_f64(g["x"], gamma, beta, N, C, HW, G, 1e-5, silu, res)
    dx, dgamma, dbeta = oracle.gn_silu_bwd_f64(g["dy"], g["x"], gamma, beta, mean, rstd,
                                               N, C, HW, G, silu, res)
    scale = np.abs(g["dx"]).max()
    np.testing.assert_allclose(dx, g["dx"].reshape(-1), rtol=1e-8, atol=1e-10 * scale)
    if affine:
        np.testing.assert_allclose(dgamma, g["dgamma"], rtol=1e-8, atol=1e-12)
        np.testing.assert_allclose(dbeta, g["dbeta"], rtol=1e-8, atol=1e-12)


def _loss(oracle, x, gamma, beta, w, N, C, HW, G, silu, res):
    y, _, _ = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, 1e-5, silu, res)
    return float(np.dot(y, w))


@pytest.mark.parametrize("silu,res", [(True, False), (False, False), (True, True)])
def test_truth_backward_finite_differences(oracle, silu, res):
    rng = np.random.default_rng(5)
    N, C, HW, G = 2, 4, 6, 2
    h = 2.0 ** -10
    # inputs on a 2^-12 grid so x +- h is exact in fp32
    q = lambda a: (np.round(a * 4096) / 4096).astype(np.float32)
    x = q(rng.standard_normal(N * C * HW))
    gamma = q(rng.uniform(0.5, 1.5, C))
    beta = q(0.1 * rng.standard_normal(C))
    w = rng.standard_normal(N * C * HW)
    _, mean, rstd = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, 1e-5, silu, res)
    dx, dgamma, dbeta = oracle.gn_silu_bwd_f64(w.astype(np.float32), x, gamma, beta, mean,
                                               rstd, N, C, HW, G, silu, res)
    # The analytic gradient used dy = fp32(w); evaluate the loss with it too.
    w32 = w.astype(np.float32).astype(np.float64)
    fd = np.empty_like(dx)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        fd[i] = (_loss(oracle, xp, gamma, beta, w32, N, C, HW, G, silu, res)
                 - _loss(oracle, xm, gamma, beta, w32, N, C, HW, G, silu, res)) / (2 * h)
    np.testing.assert_allclose(dx, fd, rtol=2e-4, atol=2e-4 * np.abs(fd).max())
    for arr, grad in ((gamma, dgamma), (beta, dbeta)):
        fdp = np.empty(C)
        for c in range(C):
            ap, am = arr.copy(), arr.copy()
            ap[c] += h
            am[c] -= h
            args_p = (ap, beta) if arr is gamma else (gamma, ap)
            args_m = (am, beta) if arr is gamma else (gamma, am)
            fdp[c] = (_loss(oracle, x, *args_p, w32, N, C, HW, G, silu, res)
                      - _loss(oracle, x, *args_m, w32, N, C, HW, G, silu, res)) / (2 * h)
        np.testing.assert_allclose(grad, fdp, rtol=2e-4, atol=2e-4 * np.abs(fdp).max())


def test_truth_closed_forms(oracle):
    N, C, HW, G = 1, 4, 16, 2
    # group 0 constant 3.0 -> var 0, rstd = 1/sqrt(eps), y = silu(beta)
    # group 1 two-valued +-2 -> mean 0, var 4
    x = np.zeros(N * C * HW, dtype=np.float32)
    x[: 2 * HW] = 3.0
    x[2 * HW:] = np.where(np.arange(2 * HW) % 2 == 0, 2.0, -2.0)
    gamma = np.array([1.0, 2.0, 0.5, 1.5], dtype=np.float32)
    beta = np.array([0.25, -0.5, 0.0, 1.0], dtype=np.float32)
    y, mean, rstd = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS32, True, False)
    assert mean[0] == 3.0 and mean[1] == 0.0
    np.testing.assert_allclose(rstd[0], 1.0 / np.sqrt(EPS32), rtol=1e-15)
    np.testing.assert_allclose(rstd[1], 1.0 / np.sqrt(4.0 + EPS32), rtol=1e-15)
    silu = lambda v: v / (1.0 + np.exp(-v))
    np.testing.assert_allclose(y[:HW], silu(0.25), rtol=1e-15)
    np.testing.assert_allclose(y[HW:2 * HW], silu(-0.5), rtol=1e-15)
    z2 = 0.5 * x[2 * HW:3 * HW] * rstd[1]
    np.testing.assert_allclose(y[2 * HW:3 * HW], silu(z2), rtol=1e-14)


def test_truth_invariants(oracle):
    rng = np.random.default_rng(9)
    N, C, HW, G = 2, 6, 50, 3
    x = rng.standard_normal(N * C * HW).astype(np.float32) * 3 + 1
    gamma = rng.uniform(0.5, 1.5, C).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = (1e-2 * rng.standard_normal(N * C * HW)).astype(np.float32)
    _, mean, rstd = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS32)
    dx, dgamma, dbeta = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mean, rstd, N, C, HW, G)
    M = (C // G) * HW
    var = 1.0 / rstd ** 2 - EPS32
    xd = x.astype(np.float64).reshape(N * G, M)
    xh = (xd - mean[:, None]) * rstd[:, None]
    dxu = dx.reshape(N * G, M)
    # sum_i dx_i = 0 per unit
    assert np.all(np.abs(dxu.sum(1)) < 1e-12 * np.abs(dxu).sum(1))
    # sum_i xhat_i dx_i = rstd*S2*eps/(var+eps), S2 = sum_c gamma_c sum dz*xhat
    xs = x.reshape(N, C, HW).astype(np.float64)
    g3 = dy.reshape(N, C, HW).astype(np.float64)
    z = gamma[None, :, None] * ((xs - np.repeat(mean.reshape(N, G), C // G, 1)[:, :, None])
                                * np.repeat(rstd.reshape(N, G), C // G, 1)[:, :, None]) \
        + beta[None, :, None]
    s = 1 / (1 + np.exp(-z))
    dz = g3 * s * (1 + z * (1 - s))
    xhat3 = (z - beta[None, :, None]) / gamma[None, :, None]
    S2 = (gamma[None, :, None] * dz * xhat3).reshape(N * G, M).sum(1)
    lhs = (xh * dxu).sum(1)
    rhs = rstd * S2 * EPS32 / (var + EPS32)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-6, atol=1e-14)
    # dy = 0 -> all gradients vanish
    z0 = np.zeros_like(dy)
    dx0, dg0, db0 = oracle.gn_silu_bwd_f64(z0, x, gamma, beta, mean, rstd, N, C, HW, G)
    assert not dx0.any() and not dg0.any() and not db0.any()
    # plain GN, gamma = 1, dy = 1: dx = r*(1 - 1 - xhat*mean(xhat)) = 0 and
    # dbeta_c = N*HW (a constant gamma is what makes dx vanish)
    ones = np.ones_like(dy)
    _, m1, r1 = oracle.gn_silu_fwd_f64(x, None, None, N, C, HW, G, EPS32, False, False)
    dx1, _, db1 = oracle.gn_silu_bwd_f64(ones, x, None, None, m1, r1, N, C, HW, G, False)
    assert np.abs(dx1).max() < 1e-12
    np.testing.assert_array_equal(db1, np.full(C, N * HW, dtype=np.float64))


def test_truth_shift_and_scale_invariance(oracle):
    rng = np.random.default_rng(3)
    N, C, HW, G = 1, 4, 64, 2
    x = rng.standard_normal(N * C * HW).astype(np.float32)
    _, m0, r0 = oracle.gn_silu_fwd_f64(x, None, None, N, C, HW, G, 0.0)
    _, m1, r1 = oracle.gn_silu_fwd_f64(x + np.float32(8.0), None, None, N, C, HW, G, 0.0)
    _, m2, r2 = oracle.gn_silu_fwd_f64(x * np.float32(4.0), None, None, N, C, HW, G, 0.0)
    np.testing.assert_allclose(m1, m0 + 8.0, rtol=1e-9, atol=1e-6)
    np.testing.assert_allclose(r1, r0, rtol=1e-6)
    np.testing.assert_allclose(m2, 4 * m0, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(r2, r0 / 4, rtol=1e-12)


# ------------------------------------------- fp32 statement of the reference

def test_reference_known_answer_input(oracle):
    """tests/test_operators.cpp:200-320: the reference's CPU formula on its own
    seeded input agrees with float64 truth within the test's 1e-4 bound."""
    k = np.load(os.path.join(GOLDEN, "kat_test_operators.npz"))
    assert int(k["mt19937_10000"][0]) == 4123659995
    x = k["x"].reshape(-1)
    assert x.min() >= -2.0 and x.max() < 2.0
    gn, means, rstds = oracle.ref_gn_forward_f32(x, k["gamma"], k["beta"], 16, 1024, 4, EPS32)
    y = oracle.ref_silu_forward_f32(gn)
    assert np.abs(y - k["y"].reshape(-1)).max() < 1e-4
    np.testing.assert_allclose(means, k["mean"], atol=1e-6)
    np.testing.assert_allclose(rstds, k["rstd"], rtol=1e-5)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, k["gamma"], k["beta"], 1, 16, 1024, 4, EPS32)
    assert np.abs(yt - k["y"].reshape(-1)).max() < 1e-6


def test_reference_port_tracks_truth(oracle):
    rng = np.random.default_rng(21)
    N, C, HW, G = 2, 8, 4096, 4
    x = rng.standard_normal(N * C * HW).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, C).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = (1e-2 * rng.standard_normal(N * C * HW)).astype(np.float32)
    r = oracle.ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, EPS32)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS32)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G)
    np.testing.assert_allclose(r["mean"], mt, atol=1e-6)
    np.testing.assert_allclose(r["rstd"], rt, rtol=1e-5)
    assert np.abs(r["y"] - yt).max() < 1e-5
    assert np.abs(r["dx"] - dxt).max() < 1e-6
    np.testing.assert_allclose(r["dgamma"], dgt, rtol=1e-3, atol=1e-5)
    np.testing.assert_allclose(r["dbeta"], dbt, rtol=1e-3, atol=1e-5)
    # residual variant: y and dx each gain exactly the residual term
    rr = oracle.ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, EPS32, residual=True)
    np.testing.assert_array_equal(rr["y"], r["y"] + x)
    np.testing.assert_array_equal(rr["dx"], r["dx"] + dy)


def test_reference_gn_backward_piecewise(oracle):
    """GroupNormNode::backward's pieces (layers.cpp:555-616) on a tiny case
    against the float64 plain-GN gradient (no SiLU)."""
    g, N, C, HW, G, silu, res, affine = case("c_plain_gn")
    x0 = g["x"][0].reshape(-1)
    dy0 = g["dy"][0].reshape(-1)
    gn, means, rstds = oracle.ref_gn_forward_f32(x0, g["gamma"], g["beta"], C, HW, G, EPS32)
    gx, gw, gb = oracle.ref_gn_backward_f32(dy0, x0, g["gamma"], means, rstds, C, HW, G)
    _, mt, rt = oracle.gn_silu_fwd_f64(x0, g["gamma"], g["beta"], 1, C, HW, G, 1e-5, False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy0, x0, g["gamma"], g["beta"], mt, rt, 1, C, HW, G,
                                           False)
    np.testing.assert_allclose(gx, dxt, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(gw, dgt, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(gb, dbt, rtol=1e-4, atol=1e-6)
    # SiLU backward piece: dsilu(v) = s(1 + v(1 - s))
    v = np.linspace(-8, 8, 33).astype(np.float32)
    got = oracle.ref_silu_backward_f32(np.ones_like(v), v)
    s = 1 / (1 + np.exp(-v.astype(np.float64)))
    np.testing.assert_allclose(got, s * (1 + v * (1 - s)), rtol=1e-5, atol=1e-7)
