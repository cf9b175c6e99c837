"""The full-size dx check (gn_checks.check_dx_correction) on the CPU: it
accepts the float64 oracle's dx rounded to fp32, and rejects dx with the
GroupNorm correction terms planted wrong (S2 dropped, sign-flipped or
halved, S1 dropped), each of which the 1e-4 value bar accepts at a unit of
2^20 elements.  The mistakes are planted in the oracle's closed form
dx = r (gamma dz - (S1 + xhat S2) / M) (src/nn/layers.cpp:606-616)."""
import numpy as np
import pytest

from gn_checks import check_dx_correction

EPS = float(np.float32(1e-5))
N, C, HW, G = 1, 8, 1 << 18, 2   # two units of 2^20 elements


@pytest.fixture(scope="module")
def case(oracle):
    seed = 20261205
    n = N * C * HW
    x = oracle.fill_normal(n, seed, 1, 0.0, 1.0)
    gamma = oracle.fill_uniform(C, seed, 2, 0.5, 1.5)
    beta = oracle.fill_normal(C, seed, 3, 0.0, 0.1)
    dy = oracle.fill_normal(n, seed, 4, 0.0, 1e-2)
    _, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, EPS, want_y=False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, N, C, HW, G)
    # the closed form's pieces, to plant mistakes in
    cpg, M = C // G, (C // G) * HW
    c = np.arange(n) // HW
    u = c // cpg
    g64 = gamma.astype(np.float64)
    xhat = (x.astype(np.float64) - mt[u]) * rt[u]
    z = g64[c] * xhat + beta[c]
    s = 1 / (1 + np.exp(-z))
    dz = dy * s * (1 + z * (1 - s))
    S1 = (g64 * dbt).reshape(G, -1).sum(1)
    S2 = (g64 * dgt).reshape(G, -1).sum(1)

    def dx_of(k1, k2):
        return rt[u] * (g64[c] * dz - (k1 * S1[u] + k2 * xhat * S2[u]) / M)

    # the closed form with the terms as they are reproduces the oracle's dx
    assert np.allclose(dx_of(1.0, 1.0), dxt, rtol=1e-12, atol=1e-18)
    return x, gamma, beta, dy, mt, rt, dxt, dx_of


def _run(case, dx64):
    import torch
    x, gamma, beta, dy, mt, rt, _, _ = case
    t = lambda a: torch.from_numpy(np.asarray(a, np.float32).reshape(N, C, HW))
    return check_dx_correction(t(dx64), t(x), t(dy), torch.from_numpy(gamma),
                               torch.from_numpy(beta), mt, rt, G, "oracle dx")


def test_accepts_the_oracle_dx_in_fp32(case):
    worst = _run(case, case[6])
    assert worst < 0.25  # fp32 rounding alone sits well inside the budget


# Each stage on its own (the others' tolerances opened up): the invariant
# sum(xhat dx) sees only the S2 term (S1 drops out of it exactly; the GPU
# tests' per-unit sum(dx) = 0 check covers S1).
STAGES = {"elementwise": ("FIT_REL", "INVARIANT_REL"),
          "fit": ("DX_ULPS", "CORR_REL", "INVARIANT_REL"),
          "invariant": ("DX_ULPS", "CORR_REL", "FIT_REL")}


MISTAKES = [(1.0, 0.0, "S2 dropped"), (1.0, -1.0, "S2 sign"), (1.0, 0.5, "S2 halved"),
            (0.0, 1.0, "S1 dropped")]


@pytest.mark.parametrize("k1,k2,what,stage", [
    m + (st,) for m in MISTAKES for st in ["all"] + list(STAGES)
    if not (st == "invariant" and m[1] == 1.0)])
def test_rejects_wrong_correction_terms(case, monkeypatch, k1, k2, what, stage):
    import gn_checks
    for name in STAGES.get(stage, ()):
        monkeypatch.setattr(gn_checks, name, 1e12)
    dxt, dx_of = case[6], case[7]
    bad = dx_of(k1, k2).astype(np.float32).astype(np.float64)
    # the value bar cannot see the mistake ...
    assert np.max(np.abs(bad - dxt) / (1 + np.abs(dxt))) <= 1e-4, what
    # ... the correction check does
    with pytest.raises(AssertionError):
        _run(case, bad)
