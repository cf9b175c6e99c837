"""HIP graph capture of the hot path.  The C-ABI entry points launch kernels
only on the stream they are given: no host synchronisation, no allocation
and no memset nodes (fills are kernels), so a GroupNorm+SiLU forward +
backward and a CBA forward + backward captured on a stream replay to the
eager results, bit for bit, every time.  Between replays the test does its
own eager work (overwriting the outputs, zeroing the accumulated gradients)
and synchronises, and it checks every replay."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GN_CASES = [
    # (N, C, HW, G): which GroupNorm path the capture holds
    (1, 64, 32 * 32, 8),        # one-launch small-unit kernels
    (2, 32, 128 * 128, 8),      # multi-kernel, finish folded into the second pass
    (1, 16, 1024 * 1024, 4),    # multi-kernel with separate finish launches
]


def _replay_and_check(g, outs, ref, reset):
    import torch
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), (rep, i)


def _capture(step):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    return g


@pytest.mark.parametrize("N,C,HW,G", GN_CASES)
def test_gn_silu_graph_replays(gpu, N, C, HW, G):
    import torch
    print(f"graph GN N={N} C={C} HW={HW} G={G}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(7 + C)
    x = torch.randn((N, C, HW), device="cuda", generator=gen)
    dy = 1e-2 * torch.randn((N, C, HW), device="cuda", generator=gen)
    gamma = 0.5 + torch.rand(C, device="cuda", generator=gen)
    beta = 0.1 * torch.randn(C, device="cuda", generator=gen)
    ws = gpu.workspace(N, C, HW, G)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    mean, rstd, lo = (torch.empty(N * G, device="cuda") for _ in range(3))
    dg, db = torch.zeros(C, device="cuda"), torch.zeros(C, device="cuda")

    def step():
        gpu.gn_silu_forward(x, gamma, beta, G, y=y, mean=mean, rstd=rstd, mean_lo=lo, ws=ws)
        gpu.gn_silu_backward(dy, x, gamma, beta, (mean, rstd, lo), G, dx=dx, dgamma=dg,
                             dbeta=db, ws=ws)

    outs = (y, mean, rstd, lo, dx, dg, db)
    step()
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]

    def reset():
        for t in (y, mean, rstd, lo, dx):
            t.fill_(float("nan"))
        dg.zero_()
        db.zero_()

    reset()
    g = _capture(step)
    _replay_and_check(g, outs, ref, reset)


CBA_CASES = [
    # (C_in, C_out, H, K): pointwise (K = 1) or depthwise CBA
    (64, 64, 128, 1),    # MFMA conv, split K, statistics in the epilogue
    (32, 64, 16, 1),     # SIMT conv, then the one-launch GroupNorm
    (32, 32, 64, 7),     # depthwise k7 (multi-tile kernels), then GroupNorm
    (256, 128, 64, 1),   # MFMA conv, K split over blocks (slices + reduce with statistics),
                         # dx reading W in place
]


@pytest.mark.parametrize("C_in,C_out,H,K", CBA_CASES)
def test_cba_graph_replays(gpu, C_in, C_out, H, K):
    import torch
    print(f"graph CBA C_in={C_in} C_out={C_out} H={H} K={K}", flush=True)
    N, HW, G = 1, H * H, 8
    gen = torch.Generator(device="cuda").manual_seed(K + H)
    x = torch.randn((N, C_in, H, H), device="cuda", generator=gen)
    dy = 1e-2 * torch.randn((N, C_out, H, H), device="cuda", generator=gen)
    gamma = 0.5 + torch.rand(C_out, device="cuda", generator=gen)
    beta = 0.1 * torch.randn(C_out, device="cuda", generator=gen)
    if K == 1:
        w = torch.randn((C_out, C_in), device="cuda", generator=gen) / C_in ** 0.5
    else:
        w = torch.randn((C_in, K, K), device="cuda", generator=gen) / K
    z = torch.empty((N, C_out, H, H), device="cuda")
    y, dz = torch.empty_like(z), torch.empty_like(z)
    mean, rstd, lo = (torch.empty(N * G, device="cuda") for _ in range(3))
    dx = torch.empty_like(x)
    dw = torch.zeros_like(w)
    dg, db = torch.zeros(C_out, device="cuda"), torch.zeros(C_out, device="cuda")
    gws = gpu.workspace(N, C_out, HW, G)
    if K == 1:
        fws = torch.empty(max(gpu.pw_conv_gn_workspace_bytes(N, C_out, HW, G), 1),
                          dtype=torch.uint8, device="cuda")
        bws = torch.empty(max(gpu.pw_conv_backward_workspace_bytes(N, C_in, C_out, HW), 1),
                          dtype=torch.uint8, device="cuda")
    else:
        n = int(gpu.lib().soar_dw_conv_backward_workspace_bytes(N, C_in, H, H, H, H, K, 1, 1))
        bws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")

    def step():
        if K == 1:
            gpu.pw_conv_gn_silu_forward(x, w, None, gamma, beta, G, eps=1e-5, z=z, y=y,
                                        mean=mean, rstd=rstd, mean_lo=lo, ws=fws)
        else:
            gpu.dw_conv_forward(x, w, None, K // 2, y=z)
            gpu.gn_silu_forward(z, gamma, beta, G, y=y, mean=mean, rstd=rstd, mean_lo=lo,
                                ws=gws)
        gpu.gn_silu_backward(dy, z, gamma, beta, (mean, rstd, lo), G, dx=dz, dgamma=dg,
                             dbeta=db, ws=gws)
        if K == 1:
            gpu.pw_conv_backward(dz, x, w, dx=dx, dweight=dw, want_db=False, ws=bws)
        else:
            gpu.dw_conv_backward(dz, x, w, K // 2, dx=dx, dweight=dw, want_db=False, ws=bws)

    outs = (z, y, mean, rstd, lo, dz, dx, dw, dg, db)
    step()
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]

    def reset():
        for t in (z, y, mean, rstd, lo, dz, dx):
            t.fill_(float("nan"))
        for t in (dw, dg, db):
            t.zero_()

    reset()
    g = _capture(step)
    _replay_and_check(g, outs, ref, reset)


@pytest.mark.parametrize("C_in,C_out,H", [(64, 64, 256), (32, 48, 128)])
def test_fused_cba_backward_graph_replays(gpu, C_in, C_out, H):
    """soar_pw_cba_backward on its fused kernel (the GroupNorm reduction and
    finish, the fused dz / dx / dW kernel, the weight-gradient finish)
    captured after the CBA forward."""
    import torch
    print(f"graph fused CBA backward C_in={C_in} C_out={C_out} H={H}", flush=True)
    N, HW, G = 1, H * H, 8
    assert N * HW >= gpu.tune_get(gpu.TUNE_PW_CBA_MIN)
    gen = torch.Generator(device="cuda").manual_seed(H + C_out)
    x = torch.randn((N, C_in, H, H), device="cuda", generator=gen)
    dy = 1e-2 * torch.randn((N, C_out, H, H), device="cuda", generator=gen)
    gamma = 0.5 + torch.rand(C_out, device="cuda", generator=gen)
    beta = 0.1 * torch.randn(C_out, device="cuda", generator=gen)
    w = torch.randn((C_out, C_in), device="cuda", generator=gen) / C_in ** 0.5
    z, y = (torch.empty((N, C_out, H, H), device="cuda") for _ in range(2))
    mean, rstd, lo = (torch.empty(N * G, device="cuda") for _ in range(3))
    dx = torch.empty_like(x)
    dw = torch.zeros_like(w)
    dg, db = torch.zeros(C_out, device="cuda"), torch.zeros(C_out, device="cuda")
    fws = torch.empty(max(gpu.pw_conv_gn_workspace_bytes(N, C_out, HW, G), 1),
                      dtype=torch.uint8, device="cuda")
    bws = torch.empty(max(gpu.pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G), 1),
                      dtype=torch.uint8, device="cuda")
    st = gpu.Stats(mean, rstd, lo)

    def step():
        gpu.pw_conv_gn_silu_forward(x, w, None, gamma, beta, G, eps=1e-5, z=z, y=y, mean=mean,
                                    rstd=rstd, mean_lo=lo, ws=fws)
        gpu.pw_cba_backward(dy, z, x, w, gamma, beta, st, G, dx=dx, dweight=dw, dgamma=dg,
                            dbeta=db, ws=bws)

    outs = (z, y, mean, rstd, lo, dx, dw, dg, db)
    step()
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]

    def reset():
        for t in (z, y, mean, rstd, lo, dx):
            t.fill_(float("nan"))
        for t in (dw, dg, db):
            t.zero_()

    reset()
    g = _capture(step)
    _replay_and_check(g, outs, ref, reset)


@pytest.mark.parametrize("K,D,H", [(3, 1, 256), (7, 1, 192), (3, 5, 160)])
def test_fused_dw_cba_backward_graph_replays(gpu, K, D, H):
    """soar_dw_cba_backward on its fused kernel (the GroupNorm reduction and
    finish, the fused dz / dx / dW kernel, the weight-gradient finish)
    captured after the depthwise CBA forward (conv, GroupNorm + SiLU)."""
    import torch
    print(f"graph fused dw CBA backward K={K} D={D} H={H}", flush=True)
    N, C, G = 1, 32, 8
    pad = (K - 1) * D // 2
    assert N * H * H >= gpu.tune_get(gpu.TUNE_DW_CBA_MIN)
    gen = torch.Generator(device="cuda").manual_seed(H + K)
    x = torch.randn((N, C, H, H), device="cuda", generator=gen)
    dy = 1e-2 * torch.randn((N, C, H, H), device="cuda", generator=gen)
    gamma = 0.5 + torch.rand(C, device="cuda", generator=gen)
    beta = 0.1 * torch.randn(C, device="cuda", generator=gen)
    w = (torch.rand((C, K, K), device="cuda", generator=gen) * 2 - 1) / K
    z, y = (torch.empty((N, C, H, H), device="cuda") for _ in range(2))
    mean, rstd, lo = (torch.empty(N * G, device="cuda") for _ in range(3))
    dx = torch.empty_like(x)
    dw = torch.zeros_like(w)
    dg, db = torch.zeros(C, device="cuda"), torch.zeros(C, device="cuda")
    fws = torch.empty(max(gpu.workspace_bytes(N, C, H * H, G), 1), dtype=torch.uint8,
                      device="cuda")
    bws = torch.empty(max(gpu.dw_cba_backward_workspace_bytes(N, C, H, H, H, H, K, pad, 1, D,
                                                              G), 1),
                      dtype=torch.uint8, device="cuda")
    st = gpu.Stats(mean, rstd, lo)

    def step():
        gpu.dw_conv_forward(x, w, None, pad, 1, D, y=z)
        gpu.gn_silu_forward(z, gamma, beta, G, eps=1e-5, y=y, mean=mean, rstd=rstd,
                            mean_lo=lo, ws=fws)
        gpu.dw_cba_backward(dy, z, x, w, gamma, beta, st, G, pad, 1, D, dx=dx, dweight=dw,
                            dgamma=dg, dbeta=db, ws=bws)

    outs = (z, y, mean, rstd, lo, dx, dw, dg, db)
    step()
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]

    def reset():
        for t in (z, y, mean, rstd, lo, dx):
            t.fill_(float("nan"))
        for t in (dw, dg, db):
            t.zero_()

    reset()
    g = _capture(step)
    _replay_and_check(g, outs, ref, reset)


NOALLOC_CASES = [
    # (C, HW, G): the multi-kernel path and the one-launch small-unit path
    (16, 256 * 256, 4),
    (16, 1024, 8),
]


def _noalloc_args(gpu, xd, dyd, gd, mean, rstd, gin, gw, gb, G, C, HW, stream):
    import ctypes
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    return (P(dyd), P(xd), P(gd), P(mean), P(rstd), P(gin), P(gw), P(gb), G, C, HW,
            ctypes.c_void_p(stream.cuda_stream))


@pytest.mark.parametrize("C,HW,G", NOALLOC_CASES)
def test_noalloc_backward_graph_replays(gpu, C, HW, G):
    """soar_group_norm_backward_noalloc captured into a graph (its workspace
    is the static scratch, whose address the library resolved at its set-up
    on this device, before the capture) replays to the eager call's results
    bit for bit, every time (the reference signature accumulates, so each
    replay starts from the same initial gradients)."""
    import torch
    print(f"graph noalloc backward C={C} HW={HW} G={G}", flush=True)
    L = gpu.lib()
    gen = torch.Generator(device="cuda").manual_seed(C + HW)
    x = torch.randn(C * HW, device="cuda", generator=gen)
    dy = 1e-2 * torch.randn(C * HW, device="cuda", generator=gen)
    gamma = 0.5 + torch.rand(C, device="cuda", generator=gen)
    beta = 0.1 * torch.randn(C, device="cuda", generator=gen)
    out = torch.empty_like(x)
    mean, rstd = torch.empty(G, device="cuda"), torch.empty(G, device="cuda")
    s0 = torch.cuda.current_stream()
    import ctypes
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    gpu.check(L.soar_group_norm_forward(P(x), P(gamma), P(beta), P(out), P(mean), P(rstd), G, C,
                                        HW, 1e-5, ctypes.c_void_p(s0.cuda_stream)))
    gin = torch.empty_like(x)
    gw, gb = torch.empty(C, device="cuda"), torch.empty(C, device="cuda")

    def reset():
        gin.fill_(0.25)
        gw.fill_(-1.0)
        gb.fill_(2.0)

    reset()
    gpu.check(L.soar_group_norm_backward_noalloc(
        *_noalloc_args(gpu, x, dy, gamma, mean, rstd, gin, gw, gb, G, C, HW, s0)))
    torch.cuda.synchronize()
    ref = [t.clone() for t in (gin, gw, gb)]
    reset()
    s = torch.cuda.Stream()

    def step():
        gpu.check(L.soar_group_norm_backward_noalloc(
            *_noalloc_args(gpu, x, dy, gamma, mean, rstd, gin, gw, gb, G, C, HW, s)))

    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    _replay_and_check(g, (gin, gw, gb), ref, reset)


_FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
import soar_gn as g
L = g.lib()
C, HW, G, eps = 16, 64 * 64, 4, 1e-5
gen = torch.Generator(device="cuda").manual_seed(5)
x = torch.randn(C * HW, device="cuda", generator=gen)
dy = 1e-2 * torch.randn(C * HW, device="cuda", generator=gen)
gamma = 0.5 + torch.rand(C, device="cuda", generator=gen)
# saved statistics from torch: no library call before the capture
xg = x.view(G, -1).double()
mean = xg.mean(1).float()
rstd = (1.0 / torch.sqrt(xg.var(1, unbiased=False) + eps)).float()
bufs = [torch.zeros(C * HW, device="cuda"), torch.zeros(C, device="cuda"),
        torch.zeros(C, device="cuda")]
P = lambda t: ctypes.c_void_p(t.data_ptr())
def call(name, stream, outs):
    return getattr(L, name)(P(dy), P(x), P(gamma), P(mean), P(rstd), *map(P, outs), G, C, HW,
                            ctypes.c_void_p(stream.cuda_stream))
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
rc = []
with torch.cuda.graph(graph, stream=s):
    rc.append(call("soar_group_norm_backward_noalloc", s, bufs))
torch.cuda.current_stream().wait_stream(s)
assert rc == [0], (rc, g.last_error())
ref = [torch.zeros_like(t) for t in bufs]
assert call("soar_group_norm_backward", torch.cuda.current_stream(), ref) == 0
for rep in range(3):
    for t in bufs:
        t.zero_()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for a, b in zip(bufs, ref):
        assert torch.equal(a, b), rep
print("FIRST_CALL_UNDER_CAPTURE_OK", flush=True)
"""


def test_noalloc_first_library_call_under_capture(gpu):
    """In a fresh process whose first call into the library is
    soar_group_norm_backward_noalloc inside a graph capture (so the scratch
    address is looked up during the capture, in relaxed capture mode): the
    capture succeeds and its replays equal soar_group_norm_backward's
    result bit for bit."""
    import os
    import subprocess
    import sys
    from conftest import ROOT
    print("noalloc first library call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE,
                        os.path.join(ROOT, "soar.cpp_amd")], capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "FIRST_CALL_UNDER_CAPTURE_OK" in r.stdout, r.stderr[-2000:]
