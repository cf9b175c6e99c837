"""Parity of the HIP path (through the C-ABI of libsoar_gn.so) against the
float64 oracle, the torch float64 fixtures and the reference's own
known-answer input.

Bars (written here, used by every check):
  stats:          |d mean| <= 1e-5 * max(|mean|, std),  |d rstd| / rstd <= 1e-5
  y, dx, dgamma, dbeta:  |d| <= 1e-4 * (1 + |truth|)
Integer/byte work (add, fill, accumulate) is checked bit-exactly.
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import GOLDEN
from gn_checks import check_dx_correction

pytestmark = pytest.mark.gpu

EPS = float(np.float32(1e-5))
STAT_TOL = 1e-5
VAL_TOL = 1e-4


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def assert_stats(mean, rstd, mean_t, rstd_t, what=""):
    mean = np.asarray(mean, np.float64)
    rstd = np.asarray(rstd, np.float64)
    std_t = np.sqrt(np.maximum(1.0 / rstd_t ** 2 - EPS, 0.0))
    dm = np.abs(mean - mean_t) / np.maximum(np.maximum(np.abs(mean_t), std_t), 1e-30)
    dr = np.abs(rstd - rstd_t) / rstd_t
    assert dm.max() <= STAT_TOL, f"{what} mean rel err {dm.max():.3e}"
    assert dr.max() <= STAT_TOL, f"{what} rstd rel err {dr.max():.3e}"


def assert_vals(got, truth, what=""):
    got = np.asarray(got, np.float64).reshape(-1)
    truth = np.asarray(truth, np.float64).reshape(-1)
    err = np.abs(got - truth) / (1.0 + np.abs(truth))
    i = int(np.argmax(err))
    assert err[i] <= VAL_TOL, f"{what} err {err[i]:.3e} at {i}: {got[i]} vs {truth[i]}"


# ----------------------------------------------------------------- fixtures

def _golden_cases():
    z = np.load(os.path.join(GOLDEN, "gn_silu_f64.npz"))
    names = sorted({k.split("/")[0] for k in z.files})
    return z, names


Z, NAMES = _golden_cases()


@pytest.mark.parametrize("name", NAMES)
def test_golden_fixture_forward_backward(gpu, name):
    g = {k.split("/")[1]: Z[k] for k in Z.files if k.startswith(name + "/")}
    N, C, HW, G, silu, res, affine = (int(v) for v in g["shape"])
    x, dy = dev(g["x"]), dev(g["dy"])
    gamma = dev(g["gamma"]) if affine else None
    beta = dev(g["beta"]) if affine else None
    y, st = gpu.gn_silu_forward(x, gamma, beta, G, eps=1e-5, silu=bool(silu),
                                        residual=bool(res))
    assert_stats(host(st.mean), host(st.rstd), g["mean"], g["rstd"], name)
    assert_vals(host(y), g["y"], name + " y")
    dx, dgamma, dbeta = gpu.gn_silu_backward(dy, x, gamma, beta, st, G,
                                             silu=bool(silu), residual=bool(res),
                                             want_params=bool(affine))
    assert_vals(host(dx), g["dx"], name + " dx")
    if affine:
        assert_vals(host(dgamma), g["dgamma"], name + " dgamma")
        assert_vals(host(dbeta), g["dbeta"], name + " dbeta")


def test_reference_known_answer(gpu):
    """tests/test_operators.cpp:200-320 of the reference: C=16, G=4, 32x32,
    gamma=1.2, beta=-0.3, mt19937(999) U(-2,2); device result within 1e-4
    absolute of the CPU formula."""
    k = np.load(os.path.join(GOLDEN, "kat_test_operators.npz"))
    x = dev(k["x"])
    y, st = gpu.gn_silu_forward(x, dev(k["gamma"]), dev(k["beta"]), 4, eps=1e-5)
    yh = host(y).reshape(-1)
    assert np.abs(yh - k["y"].reshape(-1)).max() < 1e-4
    assert_vals(yh, k["y"], "kat y")
    assert_stats(host(st.mean), host(st.rstd), k["mean"], k["rstd"], "kat")


# ------------------------------------------------------ seeded shapes vs oracle

SHAPES = [
    # (N, C, HW, G, kind)
    (1, 32, 256 * 256, 8, "normal"),       # config 1 at full size
    (1, 8, 2048 * 2048, 2, "normal"),      # config 2/3 group size (M = 2^24)
    (2, 16, 1024 * 1024, 4, "normal"),     # config 4 group size, N = 2
    (1, 4, 2048 * 2048, 1, "stress"),      # config 5 group size and input
    (3, 6, 1000, 3, "normal"),             # small planes, one chunk each
    (1, 2, 70001, 1, "normal"),            # HW % 4 != 0: scalar path, ragged chunk
    (1, 2, 70000, 2, "normal"),            # vector path, ragged last chunk
    # 300 statistics / reduction blocks and 600 apply / dx blocks: each pass
    # ends in a part-filled window of the XCD-aware block order (blocks past
    # the last whole window of 256 keep their order), and a ragged last chunk
    (1, 3, 819000, 1, "normal"),
    (2, 5, 33, 5, "normal"),               # one channel per group
    (1, 1, 1, 1, "normal"),                # single element: var = 0
    (1, 4, 1, 2, "offset"),                # HW = 1, large mean
]


def make_inputs(oracle, N, C, HW, G, kind, seed):
    n = N * C * HW
    if kind == "stress":
        x = oracle.fill_stress(n, seed)
    elif kind == "offset":
        x = oracle.fill_normal(n, seed, 1, 1e3, 1e-2)
    else:
        x = oracle.fill_normal(n, seed, 1, 0.0, 1.0)
    gamma = oracle.fill_uniform(C, seed, 2, 0.5, 1.5)
    beta = oracle.fill_normal(C, seed, 3, 0.0, 0.1)
    dy = oracle.fill_normal(n, seed, 4, 0.0, 1e-2)
    return x, gamma, beta, dy


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s[:4])) + s[4])
@pytest.mark.parametrize("residual", [False, True])
def test_seeded_shapes_vs_oracle(gpu, oracle, shape, residual):
    N, C, HW, G, kind = shape
    print(f"seeded shape N={N} C={C} HW={HW} G={G} {kind} residual={residual}", flush=True)
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, kind, 20261201 + C + HW)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, True, residual)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G, True,
                                           residual)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    y, st = gpu.gn_silu_forward(xd, dev(gamma), dev(beta), G, eps=EPS,
                                        residual=residual)
    assert_stats(host(st.mean), host(st.rstd), mt, rt, "stats")
    assert_vals(host(y), yt, "y")
    dx, dg, db = gpu.gn_silu_backward(dyd, xd, dev(gamma), dev(beta), st, G,
                                      residual=residual)
    assert_vals(host(dx), dxt, "dx")
    assert_vals(host(dg), dgt, "dgamma")
    assert_vals(host(db), dbt, "dbeta")


@pytest.mark.parametrize("silu", [False, True])
def test_no_affine_and_plain_groupnorm(gpu, oracle, silu):
    N, C, HW, G = 2, 8, 4096, 4
    x, _, _, dy = make_inputs(oracle, N, C, HW, G, "normal", 77)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, None, None, N, C, HW, G, EPS, silu, False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, None, None, mt, rt, N, C, HW, G, silu)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    y, st = gpu.gn_silu_forward(xd, None, None, G, eps=EPS, silu=silu)
    assert_vals(host(y), yt, "y")
    dx, dg, db = gpu.gn_silu_backward(dyd, xd, None, None, st, G, silu=silu)
    assert_vals(host(dx), dxt, "dx")
    assert_vals(host(dg), dgt, "dgamma")
    assert_vals(host(db), dbt, "dbeta")


def test_constant_groups(gpu):
    """var = 0 -> rstd = 1/sqrt(eps) exactly (as float), y = silu(beta)."""
    import torch
    N, C, HW, G = 1, 4, 4096, 2
    x = torch.full((N, C, HW), 3.0, device="cuda")
    beta = torch.tensor([0.25, -0.5, 0.0, 1.0], device="cuda")
    gamma = torch.ones(C, device="cuda")
    y, st = gpu.gn_silu_forward(x, gamma, beta, G, eps=EPS)
    assert np.all(host(st.mean) == 3.0)
    np.testing.assert_allclose(host(st.rstd), np.float32(1 / np.sqrt(EPS)), rtol=1e-7)
    b = beta.cpu().numpy().astype(np.float64)
    want = b / (1 + np.exp(-b))
    assert_vals(host(y)[0, :, 7], want, "y")


# --------------------------------------------- the metric config at full size

def _full_size_check(gpu, oracle, N, C, HW, G, kind, seed, samples=200000, backward=True):
    """Forward (+ backward) at a BASELINE config's full size through the
    C-ABI; stats (and dgamma/dbeta) against the oracle over the whole
    tensor, y (and dx) at sampled indices against closed forms on oracle
    statistics, and size-independent properties.  kind: "normal" (N(0,1)),
    "stress" (1e3 + N(0,1e-2) with 0.1% outliers from N(0,50)) or
    "stress_1e3" (the same with outliers from 1e3 + N(0,50))."""
    import torch
    n = N * C * HW
    print(f"full size N={N} C={C} HW={HW} G={G} {kind} backward={backward}", flush=True)
    x = torch.empty((N, C, HW), device="cuda")
    if kind == "stress":
        gpu.synth_stress(x, seed)
    elif kind == "stress_1e3":
        gpu.synth_stress(x, seed, out_mean=1e3, out_std=50.0)
    else:
        gpu.synth_normal(x, seed, 1, 0.0, 1.0)
    gamma = torch.empty(C, device="cuda")
    beta = torch.empty(C, device="cuda")
    gpu.synth_uniform(gamma, seed, 2, 0.5, 1.5)
    gpu.synth_normal(beta, seed, 3, 0.0, 0.1)
    y, st = gpu.gn_silu_forward(x, gamma, beta, G, eps=EPS)
    if not backward:
        y2, st2 = gpu.gn_silu_forward(x, gamma, beta, G, eps=EPS)
        assert torch.equal(y, y2) and all(torch.equal(a, b) for a, b in zip(st, st2))
        del y2, st2
        xh_, gh, bh = host(x).reshape(-1), host(gamma), host(beta)
        _, mt, rt = oracle.gn_silu_fwd_f64(xh_, gh, bh, N, C, HW, G, EPS, True, False,
                                           want_y=False)
        assert_stats(host(st.mean), host(st.rstd), mt, rt, "full stats")
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, n, samples)
        c = (idx // HW) % C
        u = (idx // (HW * C)) * G + c // (C // G)
        z = gh[c] * ((xh_[idx].astype(np.float64) - mt[u]) * rt[u]) + bh[c]
        assert_vals(host(y).reshape(-1)[idx], z / (1 + np.exp(-z)), "sampled y")
        return
    dy = torch.empty_like(x)
    gpu.synth_normal(dy, seed, 4, 0.0, 1e-2)
    dx, dg, db = gpu.gn_silu_backward(dy, x, gamma, beta, st, G)
    # determinism: a second run is bitwise identical
    y2, st2 = gpu.gn_silu_forward(x, gamma, beta, G, eps=EPS)
    dx2, dg2, db2 = gpu.gn_silu_backward(dy, x, gamma, beta, st2, G)
    assert torch.equal(y, y2) and all(torch.equal(a, b) for a, b in zip(st, st2))
    assert torch.equal(dx, dx2) and torch.equal(dg, dg2) and torch.equal(db, db2)
    # size-independent property: sum of dx over each unit vanishes
    dxu = dx.view(N * G, -1).double()
    assert torch.all(dxu.sum(1).abs() <= 1e-5 * dxu.abs().sum(1))
    xh_, dyh = host(x).reshape(-1), host(dy).reshape(-1)
    gh, bh = host(gamma), host(beta)
    _, mt, rt = oracle.gn_silu_fwd_f64(xh_, gh, bh, N, C, HW, G, EPS, True, False,
                                       want_y=False)
    assert_stats(host(st.mean), host(st.rstd), mt, rt, "full stats")
    _, dgt, dbt = oracle.gn_silu_bwd_f64(dyh, xh_, gh, bh, mt, rt, N, C, HW, G, want_dx=False)
    assert_vals(host(dg), dgt, "full dgamma")
    assert_vals(host(db), dbt, "full dbeta")
    # sampled y and dx from closed forms (N == 1: per-plane sums = dbeta, dgamma)
    assert N == 1
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, n, samples)
    c = idx // HW
    u = c // (C // G)
    xs = xh_[idx].astype(np.float64)
    xhat = (xs - mt[u]) * rt[u]
    z = gh[c] * xhat + bh[c]
    s = 1 / (1 + np.exp(-z))
    assert_vals(host(y).reshape(-1)[idx], z * s, "sampled y")
    dz = dyh[idx] * s * (1 + z * (1 - s))
    g64 = gh.astype(np.float64)
    S1 = (g64 * dbt).reshape(G, -1).sum(1)
    S2 = (g64 * dgt).reshape(G, -1).sum(1)
    M = (C // G) * HW
    dxt = rt[u] * (gh[c] * dz - (S1[u] + xhat * S2[u]) / M)
    assert_vals(host(dx).reshape(-1)[idx], dxt, "sampled dx")
    # every element: the correction terms with the main term taken out
    mean_eff = host(st.mean).astype(np.float64) + host(st.mean_lo).astype(np.float64)
    worst = check_dx_correction(dx, x, dy, gamma, beta, mean_eff, host(st.rstd), G,
                                f"{kind} dx")
    print(f"dx correction: largest error / bound {worst:.3f}", flush=True)


def test_full_size_config3(gpu, oracle):
    """fwd+bwd, N=1 C=64 H=W=2048 G=16, seed 20261201+3."""
    _full_size_check(gpu, oracle, 1, 64, 2048 * 2048, 16, "normal", 20261201 + 3)


def test_full_size_config5_stress(gpu, oracle):
    """x = 1e3 + N(0,1e-2), 0.1% outliers from N(0,50)."""
    _full_size_check(gpu, oracle, 1, 16, 2048 * 2048, 4, "stress", 20261201 + 5)


def test_full_size_config5_robustness(gpu, oracle):
    """Config 5's robustness variant: the outliers drawn from 1e3 + N(0,50),
    the case where the reference's fp32 CPU statistics are 6e-4 off
    (src/nn/layers.cpp:694-707)."""
    _full_size_check(gpu, oracle, 1, 16, 2048 * 2048, 4, "stress_1e3", 20261201 + 5)


def test_full_size_config2_forward(gpu, oracle):
    """BASELINE config 2 at its exact shape: forward only, N=1 C=32 H=W=2048
    G=8, seed 20261201+2."""
    _full_size_check(gpu, oracle, 1, 32, 2048 * 2048, 8, "normal", 20261201 + 2,
                     backward=False)


def test_synth_matches_oracle_generator(gpu, oracle):
    import torch
    t = torch.empty(100003, device="cuda")
    gpu.synth_normal(t, 123, 1, 0.5, 2.0)
    ref = oracle.fill_normal(t.numel(), 123, 1, 0.5, 2.0)
    # float64 libm vs device math may differ in the last bit of a double,
    # which can flip the float rounding of a rare element
    diff = np.abs(host(t) - ref)
    assert (diff > 0).mean() < 1e-3 and diff.max() < 1e-5
    gpu.synth_stress(t, 9)
    ref = oracle.fill_stress(t.numel(), 9)
    assert np.mean(host(t) == ref) > 0.999


# --------------------------------------------------------------- flags / API

def test_accumulate_semantics(gpu, oracle):
    N, C, HW, G = 1, 8, 8192, 2
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, "normal", 5)
    xd, dyd, gd, bd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW), dev(gamma), dev(beta)
    y, st = gpu.gn_silu_forward(xd, gd, bd, G, eps=EPS)
    dx1, dg, db = gpu.gn_silu_backward(dyd, xd, gd, bd, st, G)
    base = dev(np.full(N * C * HW, 0.5, np.float32)).view(N, C, HW)
    dx2, dg, db = gpu.gn_silu_backward(dyd, xd, gd, bd, st, G, dx=base,
                                       dgamma=dg, dbeta=db, accumulate_dx=True)
    np.testing.assert_allclose(host(dx2), host(dx1) + 0.5, rtol=0, atol=2e-7)
    _, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, *oracle.gn_silu_fwd_f64(
        x, gamma, beta, N, C, HW, G, EPS, want_y=False)[1:], N, C, HW, G, want_dx=False)
    assert_vals(host(dg), 2 * dgt, "dgamma x2")
    assert_vals(host(db), 2 * dbt, "dbeta x2")
    # only parameters / only dx
    none_dx, dgp, dbp = gpu.gn_silu_backward(dyd, xd, gd, bd, st, G, want_dx=False)
    assert none_dx is None
    assert_vals(host(dgp), dgt, "dgamma only")
    dxo, ng, nb = gpu.gn_silu_backward(dyd, xd, gd, bd, st, G, want_params=False)
    assert ng is None and nb is None
    assert torch_equal(dxo, dx1)


def torch_equal(a, b):
    import torch
    return torch.equal(a, b)


def test_misaligned_pointers_take_scalar_path(gpu, oracle):
    import torch
    N, C, HW, G = 1, 4, 40000, 2
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, "normal", 6)
    buf = torch.empty(N * C * HW + 1, device="cuda")
    buf[1:] = dev(x)
    xo = buf[1:].view(N, C, HW)  # 4-byte offset: not 16-byte aligned
    dbuf = torch.empty_like(buf)
    dbuf[1:] = dev(dy)
    dyo = dbuf[1:].view(N, C, HW)
    y, st = gpu.gn_silu_forward(xo, dev(gamma), dev(beta), G, eps=EPS)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS)
    assert_stats(host(st.mean), host(st.rstd), mt, rt)
    assert_vals(host(y), yt, "y")
    dx, dg, db = gpu.gn_silu_backward(dyo, xo, dev(gamma), dev(beta), st, G)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G)
    assert_vals(host(dx), dxt, "dx")
    assert_vals(host(dg), dgt, "dgamma")


def test_errors_are_statuses_not_faults(gpu):
    import torch
    L = gpu.lib()
    N, C, HW, G = 1, 4, 1024, 2
    x = torch.randn(N, C, HW, device="cuda")
    y = torch.empty_like(x)
    mean = torch.empty(N * G, device="cuda")
    rstd = torch.empty(N * G, device="cuda")
    ws = gpu.workspace(N, C, HW, G)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # workspace one byte too small
    rc = L.soar_gn_silu_forward(P(x), None, None, P(y), P(mean), P(rstd), None, N, C, HW, G, EPS,
                                1, P(ws), gpu.workspace_bytes(N, C, HW, G) - 1, s)
    assert rc == gpu.SOAR_EINVAL and "workspace" in gpu.last_error()
    # a host pointer is refused before any launch
    hx = np.zeros(N * C * HW, np.float32)
    rc = L.soar_gn_silu_forward(ctypes.c_void_p(hx.ctypes.data), None, None, P(y), P(mean),
                                P(rstd), None, N, C, HW, G, EPS, 1, P(ws), ws.numel(), s)
    assert rc == gpu.SOAR_EINVAL and "not device memory" in gpu.last_error()
    # C % G
    rc = L.soar_gn_silu_forward(P(x), None, None, P(y), P(mean), P(rstd), None, N, C, HW, 3, EPS,
                                1, P(ws), ws.numel(), s)
    assert rc == gpu.SOAR_EINVAL
    torch.cuda.synchronize()


def test_extent_check_with_arena(gpu):
    """A buffer too short for the shape is rejected (the arena gives an
    allocation whose end is known exactly)."""
    import torch
    L = gpu.lib()
    arena = ctypes.c_void_p()
    gpu.check(L.soar_arena_create(1 << 20, 256, ctypes.byref(arena)))
    try:
        p = ctypes.c_void_p()
        off = ctypes.c_size_t()
        gpu.check(L.soar_arena_alloc(arena, (1 << 20) - 4096, ctypes.byref(p),
                                     ctypes.byref(off)))
        gpu.check(L.soar_arena_alloc(arena, 4096, ctypes.byref(p), ctypes.byref(off)))
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        # 1025 floats do not fit in the last 4096 bytes
        rc = L.soar_fill(p, 1.0, 1025, s)
        assert rc == gpu.SOAR_EINVAL and "allocation holds" in gpu.last_error()
        gpu.check(L.soar_fill(p, 2.0, 1024, s))
        out = np.empty(1024, np.float32)
        gpu.check(L.soar_memcpy_d2h(ctypes.c_void_p(out.ctypes.data), p, 4096, s))
        assert np.all(out == 2.0)
    finally:
        gpu.check(L.soar_arena_destroy(arena))


def test_arena_slab_semantics(gpu):
    """tests/test_palloc_memory.cpp:74-115 of the reference: 256-byte
    alignment, static boundary, identical offsets after a dynamic reset,
    exhaustion reported."""
    L = gpu.lib()
    a = ctypes.c_void_p()
    gpu.check(L.soar_arena_create(256 * 1024 * 1024, 256, ctypes.byref(a)))
    try:
        p, off = ctypes.c_void_p(), ctypes.c_size_t()

        def alloc(n):
            gpu.check(L.soar_arena_alloc(a, n, ctypes.byref(p), ctypes.byref(off)))
            return off.value, p.value

        w1, _ = alloc(1024 * 1024 * 4)
        w2, _ = alloc(1024 * 1024 * 8 + 3)
        assert w1 % 256 == 0 and w2 % 256 == 0
        gpu.check(L.soar_arena_freeze_static(a))
        cap, cur, sb, base = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t(), \
            ctypes.c_void_p()
        gpu.check(L.soar_arena_info(a, ctypes.byref(cap), ctypes.byref(cur), ctypes.byref(sb),
                                    ctypes.byref(base)))
        assert sb.value > 0 and sb.value % 256 == 0 and cur.value == sb.value
        a1, ptr1 = alloc(512 * 512 * 64 * 2)
        a2, _ = alloc(256 * 256 * 128 * 2)
        assert a1 >= sb.value and a1 % 256 == 0 and a2 % 256 == 0
        gpu.check(L.soar_arena_reset_dynamic(a))
        gpu.check(L.soar_arena_info(a, None, ctypes.byref(cur), None, None))
        assert cur.value == sb.value
        a1b, ptr1b = alloc(512 * 512 * 64 * 2)
        assert a1b == a1 and ptr1b == ptr1
        assert L.soar_arena_alloc(a, 0, ctypes.byref(p), None) == gpu.SOAR_EINVAL
        assert L.soar_arena_alloc(a, 1 << 30, ctypes.byref(p), None) == gpu.SOAR_ENOMEM
    finally:
        gpu.check(L.soar_arena_destroy(a))


# ------------------------------------------- the reference's operator API

def test_reference_signature_group_norm(gpu, oracle):
    import torch
    L = gpu.lib()
    C, HW, G = 16, 4096, 4
    x, gamma, beta, dy = make_inputs(oracle, 1, C, HW, G, "normal", 31)
    xd, gd, bd, dyd = dev(x), dev(gamma), dev(beta), dev(dy)
    out = torch.empty_like(xd)
    mean = torch.empty(G, device="cuda")
    rstd = torch.empty(G, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gpu.check(L.soar_group_norm_forward(P(xd), P(gd), P(bd), P(out), P(mean), P(rstd), G, C,
                                        HW, EPS, s))
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, 1, C, HW, G, EPS, False)
    assert_vals(host(out), yt, "gn out")
    assert_stats(host(mean), host(rstd), mt, rt)
    # backward accumulates into pre-filled buffers (+=), gamma nullable
    gin = torch.full_like(xd, 1.0)
    gw = torch.full((C,), 2.0, device="cuda")
    gb = torch.full((C,), 3.0, device="cuda")
    gpu.check(L.soar_group_norm_backward(P(dyd), P(xd), P(gd), P(mean), P(rstd), P(gin),
                                         P(gw), P(gb), G, C, HW, s))
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, 1, C, HW, G, False)
    assert_vals(host(gin), dxt + 1.0, "grad_in +=")
    assert_vals(host(gw), dgt + 2.0, "grad_gamma +=")
    assert_vals(host(gb), dbt + 3.0, "grad_beta +=")
    # only grad_in requested
    gin2 = torch.zeros_like(xd)
    gpu.check(L.soar_group_norm_backward(P(dyd), P(xd), None, P(mean), P(rstd), P(gin2), None,
                                         None, G, C, HW, s))
    dxt1, _, _ = oracle.gn_silu_bwd_f64(dy, x, None, None, mt, rt, 1, C, HW, G, False)
    assert_vals(host(gin2), dxt1, "grad_in gamma=NULL")


def _ref_sig_fwd_bwd(gpu, x, gamma, beta, dy, C, HW, G, gin=None, gw=None, gb=None):
    """soar_group_norm_forward then soar_group_norm_backward (the reference's
    operator signatures, one sample) on host arrays; the backward adds into
    the given device buffers (None: not requested)."""
    import torch
    L = gpu.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xd, dyd = dev(x), dev(dy)
    gd = dev(gamma) if gamma is not None else None
    bd = dev(beta) if beta is not None else None
    out = torch.empty_like(xd)
    mean = torch.empty(G, device="cuda")
    rstd = torch.empty(G, device="cuda")
    gpu.check(L.soar_group_norm_forward(P(xd), P(gd), P(bd), P(out), P(mean), P(rstd), G, C,
                                        HW, EPS, s))
    gpu.check(L.soar_group_norm_backward(P(dyd), P(xd), P(gd), P(mean), P(rstd), P(gin),
                                         P(gw), P(gb), G, C, HW, s))
    return out, mean, rstd


# (C, HW, G): the small-unit kernel, a mid-size unit (the fused path would
# fold its finish), the multi-kernel path, and BASELINE config 5's shape
LARGE_MEAN_SHAPES = [(16, 1024, 8), (24, 10000, 6), (8, 256 * 256, 2),
                     (16, 2048 * 2048, 4)]


@pytest.mark.parametrize("C,HW,G", LARGE_MEAN_SHAPES, ids=lambda v: str(v))
def test_reference_signature_large_mean(gpu, oracle, C, HW, G):
    """x = 1e3 + N(0, 1e-2) through the reference-signature pair, which saves
    only the fp32 mean: the backward recovers the mean's rounding residual
    from x, so grad_in / grad_gamma / grad_beta meet the bar against the
    float64 oracle.  (With the fp32 mean alone, xhat is off by up to
    ulp(1000)/2 * rstd ~ 3e-3 and dgamma by |lo| * rstd * |sum dy| ~ 1e-2 at
    65536-pixel planes, far above the bar.)"""
    import torch
    n = C * HW
    print(f"reference-signature large mean C={C} HW={HW} G={G}", flush=True)
    seed = 20261201 + 5 + C
    x = oracle.fill_normal(n, seed, 1, 1e3, 1e-2)
    gamma = oracle.fill_uniform(C, seed, 2, 0.5, 1.5)
    beta = oracle.fill_normal(C, seed, 3, 0.0, 0.1)
    dy = oracle.fill_normal(n, seed, 4, 0.0, 1e-2)
    gin = torch.zeros(n, device="cuda")
    gw = torch.zeros(C, device="cuda")
    gb = torch.zeros(C, device="cuda")
    out, mean, rstd = _ref_sig_fwd_bwd(gpu, x, gamma, beta, dy, C, HW, G, gin, gw, gb)
    full = n <= (1 << 22)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, 1, C, HW, G, EPS, False, want_y=full)
    assert_stats(host(mean), host(rstd), mt, rt, "large-mean stats")
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, 1, C, HW, G, False,
                                           want_dx=full)
    assert_vals(host(gw), dgt, "grad_gamma")
    assert_vals(host(gb), dbt, "grad_beta")
    if full:
        assert_vals(host(out), yt, "out")
        assert_vals(host(gin), dxt, "grad_in")
    else:
        # sampled out / grad_in from closed forms on the oracle's statistics
        # and sums (one sample: the per-plane sums are dbeta and dgamma)
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, n, 200000)
        c = idx // HW
        u = c // (C // G)
        xhat = (x[idx].astype(np.float64) - mt[u]) * rt[u]
        g64 = gamma.astype(np.float64)
        assert_vals(host(out)[idx], g64[c] * xhat + beta[c], "sampled out")
        S1 = (g64 * dbt).reshape(G, -1).sum(1)
        S2 = (g64 * dgt).reshape(G, -1).sum(1)
        M = (C // G) * HW
        want = rt[u] * (g64[c] * dy[idx] - (S1[u] + xhat * S2[u]) / M)
        assert_vals(host(gin)[idx], want, "sampled grad_in")
    # every element: the correction terms with the main term taken out (the
    # backward recovers the mean's residual itself: the oracle's mean here)
    worst = check_dx_correction(gin.view(1, C, HW), dev(x).view(1, C, HW),
                                dev(dy).view(1, C, HW), dev(gamma), dev(beta), mt, host(rstd),
                                G, "large-mean grad_in", silu=False)
    print(f"grad_in correction: largest error / bound {worst:.3f}", flush=True)


@pytest.mark.parametrize("want", ["gamma", "beta", "in+gamma", "in+beta", "in", "all"])
@pytest.mark.parametrize("C,HW,G", [(16, 1024, 8), (16, 512 * 512, 8), (8, 256 * 256, 2)],
                         ids=lambda v: str(v))
def test_reference_signature_each_output_nullable(gpu, oracle, want, C, HW, G):
    """grad_in, grad_gamma and grad_beta are each optional, as the
    reference guards each (normalization_kernels.cu:142-152, 262-265): every
    combination adds exactly the requested outputs (+= onto a prefill) and
    leaves the others untouched."""
    import torch
    n = C * HW
    x, gamma, beta, dy = make_inputs(oracle, 1, C, HW, G, "normal", 61 + C)
    _, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, 1, C, HW, G, EPS, False, want_y=False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, 1, C, HW, G, False)
    parts = want.split("+") if want != "all" else ["in", "gamma", "beta"]
    gin = torch.full((n,), 0.5, device="cuda") if "in" in parts else None
    gw = torch.full((C,), -1.0, device="cuda") if "gamma" in parts else None
    gb = torch.full((C,), 2.0, device="cuda") if "beta" in parts else None
    _ref_sig_fwd_bwd(gpu, x, gamma, beta, dy, C, HW, G, gin, gw, gb)
    if gin is not None:
        assert_vals(host(gin) - 0.5, dxt, "grad_in")
    if gw is not None:
        assert_vals(host(gw) + 1.0, dgt, "grad_gamma")
    if gb is not None:
        assert_vals(host(gb) - 2.0, dbt, "grad_beta")


@pytest.mark.parametrize("which", ["dgamma", "dbeta"])
@pytest.mark.parametrize("fold", [0, 128])
def test_fused_backward_one_param_grad(gpu, oracle, restore_tuning, which, fold):
    """The fused entry point with only one of dgamma / dbeta (SiLU, saved
    mean_lo), on the folded and the separate-finish paths, with and without
    dx: the requested one accumulates, the NULL one is never touched."""
    import torch
    N, C, HW, G = 2, 32, 256 * 256, 8
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, "normal", 91)
    _, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, want_y=False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G)
    gpu.tune(gpu.TUNE_FOLD_MAX, fold)
    xd, dyd, gd, bd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW), dev(gamma), dev(beta)
    ws = gpu.workspace(N, C, HW, G)
    y, st = gpu.gn_silu_forward(xd, gd, bd, G, eps=EPS, ws=ws)
    for with_dx in (True, False):
        dx = torch.zeros_like(xd) if with_dx else None
        p = torch.full((C,), 3.0, device="cuda")
        gpu.check(gpu.lib().soar_gn_silu_backward(
            gpu._ptr(dyd), gpu._ptr(xd), gpu._ptr(gd), gpu._ptr(bd), gpu._ptr(st.mean),
            gpu._ptr(st.rstd), gpu._ptr(st.mean_lo), gpu._ptr(dx) if with_dx else None,
            gpu._ptr(p) if which == "dgamma" else None,
            gpu._ptr(p) if which == "dbeta" else None,
            N, C, HW, G, gpu.GN_SILU, gpu._ptr(ws), ws.numel(), gpu._stream()))
        assert_vals(host(p) - 3.0, dgt if which == "dgamma" else dbt, f"{which} dx={with_dx}")
        if with_dx:
            assert_vals(host(dx), dxt, "dx")


@pytest.mark.parametrize("n,offset", [(1 << 20, 0), (1001, 0), (4099, 1)])
def test_reference_signature_elementwise(gpu, oracle, n, offset):
    import torch
    L = gpu.lib()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    a_h = oracle.fill_normal(n, 3, 1, 0.0, 4.0)
    b_h = oracle.fill_normal(n, 3, 4, 0.0, 1.0)

    def buf(h):
        t = torch.empty(n + offset, device="cuda")
        t[offset:] = dev(h)
        return t[offset:]

    a, b = buf(a_h), buf(b_h)
    y = buf(np.zeros(n, np.float32))
    gpu.check(L.soar_silu_forward(P(a), P(y), n, s))
    v = a_h.astype(np.float64)
    assert_vals(host(y), v / (1 + np.exp(-v)), "silu")
    gx = buf(np.full(n, 0.25, np.float32))
    gpu.check(L.soar_silu_backward(P(b), P(a), P(gx), n, s))
    sg = 1 / (1 + np.exp(-v))
    assert_vals(host(gx), 0.25 + b_h * sg * (1 + v * (1 - sg)), "silu bwd +=")
    gpu.check(L.soar_add_forward(P(a), P(b), P(y), n, s))
    np.testing.assert_array_equal(host(y), a_h + b_h)  # one fp32 rounding: exact
    ga = buf(np.full(n, 1.5, np.float32))
    gb = buf(np.full(n, -0.5, np.float32))
    gpu.check(L.soar_add_backward(P(b), P(ga), P(gb), n, s))
    np.testing.assert_array_equal(host(ga), np.float32(1.5) + b_h)
    np.testing.assert_array_equal(host(gb), np.float32(-0.5) + b_h)
    gpu.check(L.soar_add_backward(P(b), None, P(gb), n, s))
    np.testing.assert_array_equal(host(gb), (np.float32(-0.5) + b_h) + b_h)
    gpu.check(L.soar_fill(P(y), 7.0, n, s))
    assert np.all(host(y) == 7.0)
    gpu.check(L.soar_zero(P(y), n, s))
    assert not host(y).any()


@pytest.mark.parametrize("fold", [0, 128])
def test_kernel_timing_records(gpu, restore_tuning, fold):
    import torch
    x = torch.randn(1, 8, 65536, device="cuda")
    gpu.tune(gpu.TUNE_FOLD_MAX, fold)  # the units hold 32 chunk partials
    gpu.prof_enable(True)
    try:
        y, st = gpu.gn_silu_forward(x, None, None, 2)
        gpu.gn_silu_backward(torch.randn_like(x), x, None, None, st, 2)
        recs = {r["kernel"]: r for r in gpu.prof_summary()}
    finally:
        gpu.prof_enable(False)
    # one unit batch covers this small tensor: one launch of each pass, plus
    # (without the fold) the finish-only launch of the last (here: only)
    # batch; with one batch the dx launch also finishes dgamma / dbeta, so no
    # parameter-finish launch runs either way
    passes = ["gn_stats_partial", "gn_silu_apply", "gn_silu_bwd_reduce", "gn_silu_bwd_dx"]
    finishes = ["gn_stats_finish", "gn_bwd_finish"]
    for k in passes + ([] if fold else finishes):
        assert recs[k]["launches"] == 1 and recs[k]["total_ms"] > 0
    assert "gn_param_finish" not in recs
    if fold:
        assert not set(finishes) & set(recs)


# ------------------------------------------------------------ tuning knobs

@pytest.fixture
def restore_tuning(gpu):
    keys = (gpu.TUNE_CHUNK, gpu.TUNE_REVERSE, gpu.TUNE_NT_STORE, gpu.TUNE_BATCH_MB,
            gpu.TUNE_STREAMS, gpu.TUNE_NT_LOAD, gpu.TUNE_CHUNK2, gpu.TUNE_SMALL_UNIT,
            gpu.TUNE_FOLD_MAX, gpu.TUNE_NT_TAIL_MB)
    old = {k: gpu.tune_get(k) for k in keys}
    yield
    for k, v in old.items():
        gpu.tune(k, v)


def _fwd_bwd(gpu, x, gamma, beta, dy, G, residual=False):
    N, C, HW = x.shape
    ws = gpu.workspace(N, C, HW, G)
    y, st = gpu.gn_silu_forward(x, gamma, beta, G, eps=EPS, residual=residual, ws=ws)
    dx, dg, db = gpu.gn_silu_backward(dy, x, gamma, beta, st, G, residual=residual, ws=ws)
    return [y, st.mean, st.rstd, st.mean_lo, dx, dg, db]


@pytest.mark.parametrize("residual", [False, True])
def test_tuning_variants_match(gpu, oracle, restore_tuning, residual):
    """Unit batches, streams, reverse order, load/store flavour (the first
    passes' non-temporal head / cached tail split inside the tensor with a
    1 MiB tail) and the second passes' chunking change only the launch
    schedule: results are bitwise identical to the default.  Other chunk
    sizes change the summation tree: results stay within the parity bar."""
    import torch
    N, C, HW, G = 2, 12, 65536 + 4096, 6   # unit = 2 x 69632 floats (544 KiB)
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, "normal", 41)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    gd, bd = dev(gamma), dev(beta)
    base = _fwd_bwd(gpu, xd, gd, bd, dyd, G, residual)
    for key, val in ((gpu.TUNE_BATCH_MB, 1), (gpu.TUNE_STREAMS, 2), (gpu.TUNE_BATCH_MB, 2),
                     (gpu.TUNE_NT_LOAD, 1), (gpu.TUNE_NT_LOAD, 3), (gpu.TUNE_NT_TAIL_MB, 1),
                     (gpu.TUNE_NT_TAIL_MB, 0), (gpu.TUNE_NT_LOAD, 2), (gpu.TUNE_NT_LOAD, 0),
                     (gpu.TUNE_STREAMS, 1), (gpu.TUNE_REVERSE, 0),
                     (gpu.TUNE_NT_STORE, 0), (gpu.TUNE_CHUNK2, 1024), (gpu.TUNE_CHUNK2, 16384)):
        gpu.tune(key, val)
        got = _fwd_bwd(gpu, xd, gd, bd, dyd, G, residual)
        for a, b in zip(base, got):
            assert torch.equal(a, b), (key, val)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, True, residual)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G, True,
                                           residual)
    for chunk in (1024, 4096, 16384):
        gpu.tune(gpu.TUNE_CHUNK, chunk)
        y, mean, rstd, lo, dx, dg, db = _fwd_bwd(gpu, xd, gd, bd, dyd, G, residual)
        assert_stats(host(mean), host(rstd), mt, rt, f"chunk {chunk}")
        assert_vals(host(y), yt, f"y chunk {chunk}")
        assert_vals(host(dx), dxt, f"dx chunk {chunk}")
        assert_vals(host(dg), dgt, f"dgamma chunk {chunk}")
        assert_vals(host(db), dbt, f"dbeta chunk {chunk}")


SMALL_SHAPES = [
    # (N, C, HW, G, kind): units of at most 32768 elements
    (1, 16, 1024, 8, "normal"),       # SOAR Nano, stride 2 at a 64x64 image
    (1, 256, 4, 8, "normal"),         # stride 32 at 64x64
    (1, 256, 1024, 8, "normal"),      # stride 32 at 1024x1024: unit = 32768
    (2, 64, 255, 8, "normal"),        # ragged HW, two samples
    (5, 12, 100, 4, "offset"),        # large mean, five samples walked in order
    (1, 4, 1, 2, "offset"),           # HW = 1
    (2, 4, 8000, 4, "offset"),        # 256 threads, 32 elements each: two halves in dx
    (1, 2, 30000, 2, "normal"),       # 1024 threads on one channel, two halves
]


@pytest.mark.parametrize("shape", SMALL_SHAPES, ids=lambda s: "x".join(map(str, s[:4])) + s[4])
@pytest.mark.parametrize("residual", [False, True])
def test_small_unit_path(gpu, oracle, restore_tuning, shape, residual):
    """The one-launch GroupNorm for small units against the oracle, and
    against the multi-kernel path (SOAR_TUNE_SMALL_UNIT = 0) on the same
    input, with accumulation into dx and into dgamma / dbeta."""
    import torch
    N, C, HW, G, kind = shape
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, kind, 77 + C + HW)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, True, residual)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G, True,
                                           residual)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    gd, bd = dev(gamma), dev(beta)
    runs = []
    for small in (32768, 0):
        gpu.tune(gpu.TUNE_SMALL_UNIT, small)
        y, mean, rstd, lo, dx, dg, db = _fwd_bwd(gpu, xd, gd, bd, dyd, G, residual)
        assert_stats(host(mean), host(rstd), mt, rt, f"small={small}")
        assert_vals(host(y), yt, f"y small={small}")
        assert_vals(host(dx), dxt, f"dx small={small}")
        assert_vals(host(dg), dgt, f"dgamma small={small}")
        assert_vals(host(db), dbt, f"dbeta small={small}")
        runs.append([host(t).astype(np.float64) for t in (y, dx, dg, db)])
    for a, b in zip(*runs):  # the two paths agree far inside the bar
        assert np.abs(a - b).max() <= 2e-6 * (1 + np.abs(b).max())
    # accumulation: dx += and dgamma / dbeta += (the backward's contract)
    gpu.tune(gpu.TUNE_SMALL_UNIT, 32768)
    ws = gpu.workspace(N, C, HW, G)
    y, st = gpu.gn_silu_forward(xd, gd, bd, G, eps=EPS, residual=residual, ws=ws)
    dx0 = torch.full_like(xd, 0.5)
    dg0, db0 = torch.full_like(gd, -1.0), torch.full_like(bd, 2.0)
    gpu.check(gpu.lib().soar_gn_silu_backward(
        gpu._ptr(dyd), gpu._ptr(xd), gpu._ptr(gd), gpu._ptr(bd), gpu._ptr(st.mean),
        gpu._ptr(st.rstd), gpu._ptr(st.mean_lo), gpu._ptr(dx0), gpu._ptr(dg0), gpu._ptr(db0),
        N, C, HW, G, gpu.GN_SILU | gpu.GN_ACCUMULATE_DX | (gpu.GN_RESIDUAL if residual else 0),
        gpu._ptr(ws), ws.numel(), gpu._stream()))
    assert_vals(host(dx0) - 0.5, dxt, "accumulated dx")
    assert_vals(host(dg0) + 1.0, dgt, "accumulated dgamma")
    assert_vals(host(db0) - 2.0, dbt, "accumulated dbeta")


FOLD_SHAPES = [
    # (N, C, HW, G, kind): units above 32768 elements (past the small-unit
    # kernels whatever the setting) with at most 2048 chunk partials (past
    # 128 only in units of at most 2^20 elements), so the finish folds into
    # the second pass
    (1, 16, 512 * 512, 8, "normal"),   # SOAR Nano stride 2 at 1024x1024: 64 partials
    (2, 32, 256 * 256, 8, "normal"),   # 32 partials per unit, two samples
    (1, 128, 64 * 64, 8, "normal"),    # 16 channels per group, one chunk each
    (3, 24, 10000, 6, "offset"),       # ragged chunks, large mean, three samples
    (1, 32, 512 * 512, 8, "normal"),   # 2^20-element units of a few hundred partials
]


@pytest.mark.parametrize("shape", FOLD_SHAPES, ids=lambda s: "x".join(map(str, s[:4])) + s[4])
@pytest.mark.parametrize("residual", [False, True])
def test_folded_finish(gpu, oracle, restore_tuning, shape, residual):
    """Mid-size units with the finish folded into the apply / dx pass
    (SOAR_TUNE_FOLD_MAX = 2048, the default) against the oracle, and against
    the separate finish launches (0): the statistics and y are bitwise
    identical (the same combine in the same order); dx, dgamma and dbeta
    agree far inside the bar (S1 / S2 are summed in another order); the
    parameter gradients accumulate."""
    import torch
    N, C, HW, G, kind = shape
    print(f"folded finish N={N} C={C} HW={HW} G={G} {kind} residual={residual}", flush=True)
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, kind, 5 + C)
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, True, residual)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G, True,
                                           residual)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    gd, bd = dev(gamma), dev(beta)
    runs = []
    for fold in (2048, 0):
        gpu.tune(gpu.TUNE_FOLD_MAX, fold)
        y, mean, rstd, lo, dx, dg, db = _fwd_bwd(gpu, xd, gd, bd, dyd, G, residual)
        assert_stats(host(mean), host(rstd), mt, rt, f"fold={fold}")
        assert_vals(host(y), yt, f"y fold={fold}")
        assert_vals(host(dx), dxt, f"dx fold={fold}")
        assert_vals(host(dg), dgt, f"dgamma fold={fold}")
        assert_vals(host(db), dbt, f"dbeta fold={fold}")
        runs.append([host(t) for t in (mean, rstd, lo, y, dx, dg, db)])
    for a, b in zip(runs[0][:4], runs[1][:4]):
        assert np.array_equal(a, b)
    for a, b in zip(runs[0][4:], runs[1][4:]):
        a, b = a.astype(np.float64), b.astype(np.float64)
        assert np.abs(a - b).max() <= 2e-6 * (1 + np.abs(b).max())
    # accumulation into dx and into dgamma / dbeta on the folded path
    gpu.tune(gpu.TUNE_FOLD_MAX, 2048)
    ws = gpu.workspace(N, C, HW, G)
    y, st = gpu.gn_silu_forward(xd, gd, bd, G, eps=EPS, residual=residual, ws=ws)
    dx0 = torch.full_like(xd, 0.5)
    dg0, db0 = torch.full_like(gd, -1.0), torch.full_like(bd, 2.0)
    gpu.check(gpu.lib().soar_gn_silu_backward(
        gpu._ptr(dyd), gpu._ptr(xd), gpu._ptr(gd), gpu._ptr(bd), gpu._ptr(st.mean),
        gpu._ptr(st.rstd), gpu._ptr(st.mean_lo), gpu._ptr(dx0), gpu._ptr(dg0), gpu._ptr(db0),
        N, C, HW, G, gpu.GN_SILU | gpu.GN_ACCUMULATE_DX | (gpu.GN_RESIDUAL if residual else 0),
        gpu._ptr(ws), ws.numel(), gpu._stream()))
    assert_vals(host(dx0) - 0.5, dxt, "accumulated dx")
    assert_vals(host(dg0) + 1.0, dgt, "accumulated dgamma")
    assert_vals(host(db0) - 2.0, dbt, "accumulated dbeta")


def test_full_size_config4_chain(gpu, oracle):
    """six SOAR blocks x <- x + silu(gn(x)) at N=2, C=128,
    H=W=1024, G=32, forward then backward, fused (SOAR_GN_RESIDUAL).
    Every block: dgamma/dbeta over the whole tensor against the oracle fed
    with that block's device input and upstream gradient (per sample, which
    also gives the per-unit sums S1 / S2); sum over each unit of (dx - dy)
    vanishes; the output at sampled indices against closed forms; for the
    first and last blocks, dx at sampled indices against the closed form
    dx = rstd*(gamma*dz - (S1 + xhat*S2)/M) + dy on oracle statistics and
    sums; for every block, every element's correction terms
    (gn_checks.check_dx_correction)."""
    import torch
    N, C, HW, G, B = 2, 128, 1024 * 1024, 32, 6
    seed = 20261201 + 4
    x0 = torch.empty((N, C, HW), device="cuda")
    gpu.synth_normal(x0, seed, 1, 0.0, 1.0)
    dy = torch.empty_like(x0)
    gpu.synth_normal(dy, seed, 4, 0.0, 1e-2)
    params = []
    for b in range(B):
        g = torch.empty(C, device="cuda")
        be = torch.empty(C, device="cuda")
        gpu.synth_uniform(g, seed + 1000 * b, 2, 0.5, 1.5)
        gpu.synth_normal(be, seed + 1000 * b, 3, 0.0, 0.1)
        params.append((g, be))
    ws = gpu.workspace(N, C, HW, G)
    acts, stats = [x0], []
    for b in range(B):
        y, st = gpu.gn_silu_forward(acts[-1], *params[b], G, eps=EPS, residual=True, ws=ws)
        acts.append(y)
        stats.append(st)
    g_in = dy
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, N * C * HW, 100000)
    for b in reversed(range(B)):
        dx, dg, db = gpu.gn_silu_backward(g_in, acts[b], *params[b], stats[b], G, residual=True,
                                          ws=ws)
        # sum over each unit of dx - dy = sum of the GroupNorm part = 0
        d = (dx - g_in).view(N * G, -1).double()
        assert torch.all(d.sum(1).abs() <= 1e-5 * d.abs().sum(1)), b
        xh, gh = host(acts[b]).reshape(-1), host(g_in).reshape(-1)
        gm, bt = host(params[b][0]), host(params[b][1])
        print(f"config 4 chain block {b}", flush=True)
        _, mt, rt = oracle.gn_silu_fwd_f64(xh, gm, bt, N, C, HW, G, EPS, True, True,
                                           want_y=False)
        assert_stats(host(stats[b].mean), host(stats[b].rstd), mt, rt, f"block {b}")
        # per sample: that sample's per-plane sums of dz*xhat and dz
        S = C * HW
        per = [oracle.gn_silu_bwd_f64(gh[k * S:(k + 1) * S], xh[k * S:(k + 1) * S], gm, bt,
                                      mt[k * G:(k + 1) * G], rt[k * G:(k + 1) * G], 1, C, HW,
                                      G, True, True, want_dx=False)[1:] for k in range(N)]
        dgt = sum(p[0] for p in per)
        dbt = sum(p[1] for p in per)
        assert_vals(host(dg), dgt, f"block {b} dgamma")
        assert_vals(host(db), dbt, f"block {b} dbeta")
        c = (idx // HW) % C
        nn_ = idx // (HW * C)
        u = nn_ * G + c // (C // G)
        xs = xh[idx].astype(np.float64)
        xhat = (xs - mt[u]) * rt[u]
        z = gm[c] * xhat + bt[c]
        sg = 1 / (1 + np.exp(-z))
        assert_vals(host(acts[b + 1]).reshape(-1)[idx], xs + z * sg, f"block {b} y")
        if b in (0, B - 1):
            g64 = gm.astype(np.float64)
            S1 = np.concatenate([(g64 * p[1]).reshape(G, -1).sum(1) for p in per])
            S2 = np.concatenate([(g64 * p[0]).reshape(G, -1).sum(1) for p in per])
            M = (C // G) * HW
            gs = gh[idx].astype(np.float64)
            dz = gs * sg * (1 + z * (1 - sg))
            want = rt[u] * (g64[c] * dz - (S1[u] + xhat * S2[u]) / M) + gs
            assert_vals(host(dx).reshape(-1)[idx], want, f"block {b} sampled dx")
        # every element of every block: the correction terms
        st = stats[b]
        mean_eff = host(st.mean).astype(np.float64) + host(st.mean_lo).astype(np.float64)
        worst = check_dx_correction(dx, acts[b], g_in, *params[b], mean_eff, host(st.rstd), G,
                                    f"block {b} dx", residual=True)
        print(f"block {b} dx correction: largest error / bound {worst:.3f}", flush=True)
        del xh, gh
        g_in = dx
