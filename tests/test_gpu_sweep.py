"""Seeded sweep of the fused GroupNorm(+SiLU) path against the float64 oracle.

Each case draws its shape (N, C = G * cpg, HW), input kind, flags (SiLU,
residual, accumulate into dx), affine parameters (both, none, or one of
them), whether the forward saves the mean residual, and the launch tuning
(chunk sizes, the one-launch small-unit path, the folded finish, loads in
flight, unit batching) from one generator, so the interactions the
hand-written tests do not enumerate are covered by a fixed, repeatable set.
Every case runs the forward and the backward through the C-ABI and checks
them with the bars of tests/test_gpu_parity.py:
  stats:          |d mean| <= 1e-5 * max(|mean|, std),  |d rstd| / rstd <= 1e-5
  y, dx, dgamma, dbeta:  |d| <= 1e-4 * (1 + |truth|)
(dx when accumulating: the sum's truth is base + dx, and the bar is taken on
it.)

A second sweep does the same for the CBA block with a pointwise conv (the
conv with the GroupNorm statistics in its epilogue, then the GroupNorm
backward on z and the conv backward), under random choices of the SIMT /
MFMA paths, the split over blocks and the weight gradient's waves per
block, with the bars of tests/test_gpu_pw_conv.py for z, dx, dW and db.
"""
import numpy as np
import pytest

from test_gpu_parity import EPS, assert_stats, assert_vals, dev, host, make_inputs
from test_gpu_pw_conv import assert_z, bwd_bounds, rng_inputs

pytestmark = pytest.mark.gpu

HWS = [1, 2, 3, 17, 64, 255, 1000, 4097, 16385, 70001, 131072]
CPGS = [1, 2, 3, 4, 5, 8]
KINDS = ["normal", "normal", "offset", "stress"]
CHUNKS = [(1024, 1024), (4096, 4096), (8192, 4096), (16384, 8192)]


def _cases(n_cases=96, seed=20261202):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        N = int(r.integers(1, 4))
        G = int(r.integers(1, 9))
        cpg = int(r.choice(CPGS))
        HW = int(r.choice(HWS))
        C = G * cpg
        if N * C * HW > 3_000_000:
            continue
        kind = str(r.choice(KINDS))
        silu = bool(r.integers(0, 2))
        residual = bool(r.integers(0, 2))
        accumulate = bool(r.integers(0, 2))
        affine = str(r.choice(["both", "both", "none", "gamma", "beta"]))
        # without the saved residual only the plain GroupNorm recovers it
        # (with SiLU at a large mean that is the reference's precision)
        keep_lo = True if (silu and kind != "normal") else bool(r.integers(0, 2))
        chunk, chunk2 = CHUNKS[int(r.integers(0, len(CHUNKS)))]
        tune = {"chunk": chunk, "chunk2": chunk2,
                "small_unit": int(r.choice([0, 16384])),
                "fold_max": int(r.choice([0, 128])),
                "loads": int(r.choice([4, 8])),
                "batch_mb": int(r.choice([0, 0, 1]))}
        out.append((N, C, HW, G, kind, silu, residual, accumulate, affine, keep_lo, tune))
    return out


CASES = _cases()


def _id(c):
    N, C, HW, G, kind, silu, res, acc, aff, lo, t = c
    return (f"{N}x{C}x{HW}g{G}-{kind}-{'silu' if silu else 'gn'}{'-res' if res else ''}"
            f"{'-acc' if acc else ''}-{aff}{'' if lo else '-nolo'}-c{t['chunk']}"
            f"-s{t['small_unit']}-f{t['fold_max']}-l{t['loads']}-b{t['batch_mb']}")


@pytest.fixture
def tuning(gpu):
    keys = {"chunk": gpu.TUNE_CHUNK, "chunk2": gpu.TUNE_CHUNK2,
            "small_unit": gpu.TUNE_SMALL_UNIT, "fold_max": gpu.TUNE_FOLD_MAX,
            "loads": gpu.TUNE_LOADS, "batch_mb": gpu.TUNE_BATCH_MB}
    old = {k: gpu.tune_get(v) for k, v in keys.items()}

    def apply(t):
        for k, v in t.items():
            gpu.tune(keys[k], v)

    yield apply
    apply(old)


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_sweep_vs_oracle(gpu, oracle, tuning, case):
    N, C, HW, G, kind, silu, residual, accumulate, affine, keep_lo, tune = case
    print(f"sweep {_id(case)}", flush=True)
    tuning(tune)
    x, gamma, beta, dy = make_inputs(oracle, N, C, HW, G, kind, 7 * HW + 13 * C + N)
    g = gamma if affine in ("both", "gamma") else None
    b = beta if affine in ("both", "beta") else None
    yt, mt, rt = oracle.gn_silu_fwd_f64(x, g, b, N, C, HW, G, EPS, silu, residual)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, g, b, mt, rt, N, C, HW, G, silu, residual)
    xd, dyd = dev(x).view(N, C, HW), dev(dy).view(N, C, HW)
    gd = dev(g) if g is not None else None
    bd = dev(b) if b is not None else None
    y, st = gpu.gn_silu_forward(xd, gd, bd, G, eps=EPS, silu=silu, residual=residual,
                                keep_lo=keep_lo)
    assert_stats(host(st.mean), host(st.rstd), mt, rt, "stats")
    assert_vals(host(y), yt, "y")
    base = None
    dx_in = None
    if accumulate:
        base = np.random.default_rng(HW).standard_normal((N, C, HW)).astype(np.float32)
        dx_in = dev(base)
    dx, dgm, dbt_d = gpu.gn_silu_backward(dyd, xd, gd, bd, st, G, silu=silu,
                                          residual=residual, dx=dx_in,
                                          accumulate_dx=accumulate)
    if accumulate:
        assert_vals(host(dx), base.astype(np.float64).reshape(-1) + dxt, "dx (accumulated)")
    else:
        assert_vals(host(dx), dxt, "dx")
    assert_vals(host(dgm), dgt, "dgamma")
    assert_vals(host(dbt_d), dbt, "dbeta")


# ---- CBA with a pointwise conv ---------------------------------------------------

def _cba_cases(n_cases=32, seed=20261203):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        N = int(r.integers(1, 3))
        G = int(r.choice([1, 2, 4, 8, 16]))
        C_out = G * int(r.choice([1, 2, 4, 6]))
        C_in = int(r.choice([1, 3, 8, 16, 24, 64, 130, 256]))
        HW = int(r.choice([1, 7, 64, 333, 1024, 2500, 4096, 16384]))
        if N * max(C_in, C_out) * HW > 2_000_000 or N * C_in * C_out * HW > 2e9:
            continue
        kind = str(r.choice(["normal", "normal", "offset"]))
        silu = bool(r.integers(0, 2))
        tune = {"pw_small": int(r.choice([0, 1 << 25])), "pw_splitk": int(r.choice([1, 8])),
                "pw_wg_waves": int(r.choice([1, 4, 8])), "pw_chunk": int(r.choice([512, 1024]))}
        out.append((N, C_in, C_out, HW, G, kind, silu, tune))
    return out


CBA_CASES = _cba_cases()


def _cba_id(c):
    N, C_in, C_out, HW, G, kind, silu, t = c
    return (f"{N}x{C_in}to{C_out}x{HW}g{G}-{kind}-{'silu' if silu else 'gn'}"
            f"-s{t['pw_small']}-k{t['pw_splitk']}-w{t['pw_wg_waves']}-c{t['pw_chunk']}")


@pytest.fixture
def pw_tuning(gpu):
    keys = {"pw_small": gpu.TUNE_PW_SMALL, "pw_splitk": gpu.TUNE_PW_SPLITK,
            "pw_wg_waves": gpu.TUNE_PW_WG_WAVES, "pw_chunk": gpu.TUNE_PW_CHUNK}
    old = {k: gpu.tune_get(v) for k, v in keys.items()}

    def apply(t):
        for k, v in t.items():
            gpu.tune(keys[k], v)

    yield apply
    apply(old)


@pytest.mark.parametrize("case", CBA_CASES, ids=_cba_id)
def test_cba_sweep_vs_oracle(gpu, oracle, pw_tuning, case):
    N, C_in, C_out, HW, G, kind, silu, tune = case
    print(f"cba sweep {_cba_id(case)}", flush=True)
    pw_tuning(tune)
    x, w, b = rng_inputs(HW + C_in + 5 * C_out, N, C_in, C_out, HW, True, kind)
    r = np.random.default_rng(C_out + HW)
    gamma = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    beta = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    dy = (1e-2 * r.standard_normal((N, C_out, HW))).astype(np.float32)
    xd, wd, gd, bd = dev(x), dev(w), dev(gamma), dev(beta)
    z, y, st = gpu.pw_conv_gn_silu_forward(xd, wd, dev(b), gd, bd, G, eps=EPS, silu=silu)
    zh = host(z)
    assert_z(zh, x, w, b, oracle, "z")
    y_t, mean_t, rstd_t = oracle.gn_silu_fwd_f64(zh, gamma, beta, N, C_out, HW, G, EPS,
                                                 silu=silu)
    assert_stats(host(st.mean), host(st.rstd), mean_t, rstd_t, "stats")
    assert_vals(host(y), y_t, "y")
    # GroupNorm backward on z with the saved statistics, then the conv's
    dz, dgm, dbt = gpu.gn_silu_backward(dev(dy), z, gd, bd, st, G, silu=silu)
    dz_t, dg_t, db_t = oracle.gn_silu_bwd_f64(dy, zh, gamma, beta, mean_t, rstd_t, N, C_out,
                                              HW, G, silu)
    assert_vals(host(dz), dz_t, "dz")
    assert_vals(host(dgm), dg_t, "dgamma")
    assert_vals(host(dbt), db_t, "dbeta")
    dzh = host(dz)
    dx, dw, db = gpu.pw_conv_backward(dz, xd, wd)
    tx, tw, tb = oracle.conv1x1_bwd_f64(dzh, x, w, N, C_in, C_out, HW)
    bx, bw, bb = bwd_bounds(dzh, x, w)
    for got, t, bnd, name in ((dx, tx, bx, "dx"), (dw, tw, bw, "dw"), (db, tb, bb, "db")):
        err = np.abs(host(got).astype(np.float64).reshape(-1) - t)
        ratio = err / (bnd.reshape(-1) + 1e-30)
        i = int(np.argmax(ratio))
        assert ratio[i] <= 1.0, f"{name} err {err[i]:.3e} > bound {bnd.reshape(-1)[i]:.3e}"
    # the fused CBA backward (soar_pw_cba_backward; its fused kernel wherever
    # C_in and C_out are multiples of 8 up to 64 and HW % 4 == 0, else the
    # two calls above), against
    # the stand-alone GroupNorm backward's dz on its multi-kernel path, whose
    # reduction and dx arithmetic the fused kernel shares
    keys = (gpu.TUNE_PW_CBA_MIN, gpu.TUNE_SMALL_UNIT, gpu.TUNE_FOLD_MAX)
    old = {k: gpu.tune_get(k) for k in keys}
    try:
        gpu.tune(gpu.TUNE_PW_CBA_MIN, 1)
        gpu.tune(gpu.TUNE_SMALL_UNIT, 0)
        gpu.tune(gpu.TUNE_FOLD_MAX, 0)
        dz2, dg2, db2 = gpu.gn_silu_backward(dev(dy), z, gd, bd, st, G, silu=silu)
        fx, fw, fg, fb = gpu.pw_cba_backward(dev(dy), z, xd, wd, gd, bd, st, G, silu=silu)
    finally:
        for k, v in old.items():
            gpu.tune(k, v)
    assert np.array_equal(host(fg), host(dg2)) and np.array_equal(host(fb), host(db2))
    dzh2 = host(dz2)
    tx, tw, _ = oracle.conv1x1_bwd_f64(dzh2, x, w, N, C_in, C_out, HW, want=("dx", "dw"))
    bx, bw, _ = bwd_bounds(dzh2, x, w)
    for got, t, bnd, name in ((fx, tx, bx, "fused dx"), (fw, tw, bw, "fused dw")):
        err = np.abs(host(got).astype(np.float64).reshape(-1) - t)
        ratio = err / (bnd.reshape(-1) + 1e-30)
        i = int(np.argmax(ratio))
        assert ratio[i] <= 1.0, f"{name} err {err[i]:.3e} > bound {bnd.reshape(-1)[i]:.3e}"
