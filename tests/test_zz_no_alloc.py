"""soar_group_norm_backward_noalloc, the allocation-free variant of the
reference-signature GroupNorm backward (its workspace is a static device
array), against soar_group_norm_backward on the same inputs: bitwise equal
results (same kernels, same plan), on consecutive calls whose inputs shrink,
so the second call runs over what the first left in the shared scratch.
Both are also held to the float64 oracle at the parity bar
|d| <= 1e-4 * (1 + |truth|)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS = float(np.float32(1e-5))
VAL_TOL = 1e-4


def _assert_vals(got, truth, what):
    got = np.asarray(got, np.float64).reshape(-1)
    truth = np.asarray(truth, np.float64).reshape(-1)
    err = np.abs(got - truth) / (1.0 + np.abs(truth))
    assert err.max() <= VAL_TOL, f"{what} err {err.max():.3e}"


def _compare(gpu, oracle, C, HW, G, seed, kind):
    import torch
    L = gpu.lib()
    n = C * HW
    print(f"noalloc vs group_norm_backward C={C} HW={HW} G={G} {kind}", flush=True)
    mu, sd = (1e3, 1e-2) if kind == "offset" else (0.0, 1.0)
    x = oracle.fill_normal(n, seed, 1, mu, sd)
    gamma = oracle.fill_uniform(C, seed, 2, 0.5, 1.5)
    beta = oracle.fill_normal(C, seed, 3, 0.0, 0.1)
    dy = oracle.fill_normal(n, seed, 4, 0.0, 1e-2)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    xd, gd, bd, dyd = dev(x), dev(gamma), dev(beta), dev(dy)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.empty_like(xd)
    mean = torch.empty(G, device="cuda")
    rstd = torch.empty(G, device="cuda")
    gpu.check(L.soar_group_norm_forward(P(xd), P(gd), P(bd), P(out), P(mean), P(rstd), G, C,
                                        HW, EPS, s))
    results = []
    for name in ("soar_group_norm_backward", "soar_group_norm_backward_noalloc"):
        gin = torch.full((n,), 0.5, device="cuda")
        gw = torch.full((C,), -1.0, device="cuda")
        gb = torch.full((C,), 2.0, device="cuda")
        gpu.check(getattr(L, name)(P(dyd), P(xd), P(gd), P(mean), P(rstd), P(gin), P(gw),
                                   P(gb), G, C, HW, s))
        torch.cuda.synchronize()
        results.append((gin, gw, gb))
    for a, b, what in zip(results[0], results[1], ("grad_in", "grad_gamma", "grad_beta")):
        assert torch.equal(a, b), what
    _, mt, rt = oracle.gn_silu_fwd_f64(x, gamma, beta, 1, C, HW, G, EPS, False, want_y=False)
    dxt, dgt, dbt = oracle.gn_silu_bwd_f64(dy, x, gamma, beta, mt, rt, 1, C, HW, G, False)
    gin, gw, gb = (t.cpu().numpy() for t in results[1])
    _assert_vals(gin - 0.5, dxt, "grad_in")
    _assert_vals(gw + 1.0, dgt, "grad_gamma")
    _assert_vals(gb - 2.0, dbt, "grad_beta")


def test_noalloc_matches_group_norm_backward(gpu, oracle):
    # large mean first (the mean residual recovery uses the most scratch
    # regions), then smaller inputs over the same scratch: the multi-kernel
    # path, then the one-launch small-unit path
    _compare(gpu, oracle, 16, 1024 * 1024, 4, 20261211, "offset")
    _compare(gpu, oracle, 8, 256 * 256, 2, 20261212, "normal")
    _compare(gpu, oracle, 16, 1024, 8, 20261213, "normal")


def test_noalloc_refuses_shapes_beyond_the_scratch(gpu):
    import torch
    L = gpu.lib()
    C, HW, G = 512, 2048 * 2048, 8
    need = gpu.workspace_bytes(1, C, HW, G)
    assert need > gpu.NOALLOC_SCRATCH_BYTES
    t = torch.zeros(16, device="cuda")
    P = ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.soar_group_norm_backward_noalloc(P, P, None, P, P, P, None, None, G, C, HW, s)
    assert rc == gpu.SOAR_EINVAL and "static scratch" in gpu.last_error()
    torch.cuda.synchronize()
    assert not t.any()
