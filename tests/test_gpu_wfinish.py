"""Deferred weight-gradient finishes (SOAR_DEFER_WEIGHT_FINISH and
soar_weight_grad_flush) through the C-ABI of libsoar_gn.so.

A convolution backward call with the flag leaves its weight / bias
gradient partials in its workspace and queues the finish; the flush adds
every queued finish in one launch with the same float64 sums in the same
order as the call's own finish.  Each case checks:
  before the flush: dweight / dbias untouched (still the caller's values),
                    dx written, the queue holding the call's entries;
  after the flush:  dweight / dbias bit for bit equal to an immediate call
                    on the same inputs (and the queue empty);
for the pointwise and depthwise (k3, k7, stride 2) convolution backward and
the pointwise / depthwise CBA backward, alone and queued together; two calls
into one dweight (the second flushes the first: their additions would race
in one launch); a discard (the pending finishes of an abandoned pass never
run); a flush on another stream (refused); and a captured graph of
deferred backward calls and the flush, replayed with eager work between the
replays, against the same calls run eagerly.
"""
import numpy as np
import pytest

from test_gpu_parity import EPS

pytestmark = pytest.mark.gpu


def _rand(gen, *shape, scale=1.0):
    import torch
    return scale * torch.randn(shape, generator=gen, device="cuda")


def _ws(nbytes):
    """A workspace of its own for one call (a deferred call's partials stay
    in it until the flush, so every call here gets a fresh one and the
    caller keeps it)."""
    import torch
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device="cuda")


def _pw_case(gpu, gen, N=2, C_in=24, C_out=40, H=96, W=96):
    # (N*H*W above 16384: the split-K weight gradient with its finish, not
    # the one-launch small kernel)
    x = _rand(gen, N, C_in, H, W)
    w = _rand(gen, C_out, C_in, scale=0.2)
    dz = _rand(gen, N, C_out, H, W, scale=1e-2)

    def run(defer, dw, db, ws=None):
        ws = _ws(gpu.pw_conv_backward_workspace_bytes(N, C_in, C_out, H * W)) if ws is None else ws
        r = gpu.pw_conv_backward(dz, x, w, dweight=dw, dbias=db, ws=ws, defer_finish=defer)
        return r[0], ws
    return run, (C_out, C_in), C_out


def _dw_case(gpu, gen, K=3, S=1, N=2, C=16, H=70, W=66):
    import torch
    pad = (K - 1) // 2
    x = _rand(gen, N, C, H, W)
    w = _rand(gen, C, K, K, scale=1.0 / K)
    Ho = (H + 2 * pad - K) // S + 1
    Wo = (W + 2 * pad - K) // S + 1
    dy = _rand(gen, N, C, Ho, Wo, scale=1e-2)
    del torch

    def run(defer, dw, db, ws=None):
        if ws is None:
            ws = _ws(gpu.lib().soar_dw_conv_backward_workspace_bytes(N, C, H, W, Ho, Wo, K, S, 1))
        r = gpu.dw_conv_backward(dy, x, w, pad, S, dweight=dw, dbias=db, ws=ws,
                                 defer_finish=defer)
        return r[0], ws
    return run, (C, K, K), C


def _pw_cba_case(gpu, gen, N=2, C_in=64, C_out=64, H=128, W=128, G=16):
    x = _rand(gen, N, C_in, H, W)
    w = _rand(gen, C_out, C_in, scale=0.125)
    gm = 1.0 + _rand(gen, C_out, scale=0.1)
    bt = _rand(gen, C_out, scale=0.1)
    dy = _rand(gen, N, C_out, H, W, scale=1e-2)
    z, _, st = gpu.pw_conv_gn_silu_forward(x, w, None, gm, bt, G, eps=EPS)

    def run(defer, dw, db, ws=None):
        ws = _ws(gpu.pw_cba_backward_workspace_bytes(N, C_in, C_out, H * W, G)) if ws is None else ws
        r = gpu.pw_cba_backward(dy, z, x, w, gm, bt, st, G, dweight=dw, want_params=False,
                                ws=ws, defer_finish=defer)
        return r[0], ws
    return run, (C_out, C_in), None


def _dw_cba_case(gpu, gen, K=7, N=2, C=16, H=160, W=130, G=4):
    pad = (K - 1) // 2
    x = _rand(gen, N, C, H, W)
    w = _rand(gen, C, K, K, scale=1.0 / K)
    gm = 1.0 + _rand(gen, C, scale=0.1)
    bt = _rand(gen, C, scale=0.1)
    dy = _rand(gen, N, C, H, W, scale=1e-2)
    z, _, st = gpu.dw_conv_gn_silu_forward(x, w, None, gm, bt, G, pad, eps=EPS)

    def run(defer, dw, db, ws=None):
        if ws is None:
            ws = _ws(gpu.dw_cba_backward_workspace_bytes(N, C, H, W, H, W, K, pad, 1, 1, G))
        r = gpu.dw_cba_backward(dy, z, x, w, gm, bt, st, G, pad, dweight=dw, want_params=False,
                                ws=ws, defer_finish=defer)
        return r[0], ws
    return run, (C, K, K), None


CASES = {
    "pw": _pw_case,
    # few partials per element (the finish's one-element-per-thread path)
    "pw_narrow": lambda g, r: _pw_case(g, r, N=1, C_in=128, C_out=256, H=32, W=32),
    # many partials per element (a wave per segment)
    "dw_k3_wide": lambda g, r: _dw_case(g, r, K=3, N=2, C=8, H=256, W=256),
    "dw_k3": lambda g, r: _dw_case(g, r, K=3),
    "dw_k7": lambda g, r: _dw_case(g, r, K=7),
    "dw_k3_s2": lambda g, r: _dw_case(g, r, K=3, S=2),
    "pw_cba": _pw_cba_case,
    "dw_cba_k7": _dw_cba_case,
}


def _grads(wshape, bsize, seed):
    """Pre-filled gradient buffers: the finishes add into them."""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dw = _rand(gen, *wshape, scale=1e-3)
    db = _rand(gen, bsize, scale=1e-3) if bsize else None
    return dw, db


def _eq(a, b):
    import torch
    return a is None and b is None or torch.equal(a, b)


@pytest.mark.parametrize("name", list(CASES))
def test_deferred_finish_matches_immediate(gpu, name):
    import torch
    print(f"deferred weight finish: {name}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261210 + len(name))
    run, wshape, bsize = CASES[name](gpu, gen)
    dw0, db0 = _grads(wshape, bsize, 7)
    dwi, dbi = dw0.clone(), (db0.clone() if db0 is not None else None)
    dxi, _ = run(False, dwi, dbi)
    dwd, dbd = dw0.clone(), (db0.clone() if db0 is not None else None)
    assert gpu.weight_grad_pending() == 0
    dxd, ws = run(True, dwd, dbd)
    torch.cuda.synchronize()
    queued = gpu.weight_grad_pending()
    assert queued >= 1
    assert torch.equal(dxd, dxi)  # dx at once
    assert torch.equal(dwd, dw0) and _eq(dbd, db0)  # the weights wait for the flush
    gpu.weight_grad_flush()
    torch.cuda.synchronize()
    assert gpu.weight_grad_pending() == 0
    assert torch.equal(dwd, dwi) and _eq(dbd, dbi)
    del ws


def test_queued_together_one_flush(gpu):
    """Every case queued before one flush (each in its own workspace)."""
    import torch
    print("deferred weight finish: all cases, one flush", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261211)
    cases = [CASES[n](gpu, gen) for n in CASES]
    imm, dfr = [], []
    for i, (run, wshape, bsize) in enumerate(cases):
        dw0, db0 = _grads(wshape, bsize, 100 + i)
        a = (dw0.clone(), db0.clone() if db0 is not None else None)
        run(False, *a)
        imm.append(a)
        dfr.append((dw0.clone(), db0.clone() if db0 is not None else None))
    kept = []  # the workspaces stay alive until the flush
    for (run, wshape, bsize), (dw, db) in zip(cases, dfr):
        kept.append(run(True, dw, db))
    assert gpu.weight_grad_pending() >= len(cases)
    gpu.weight_grad_flush()
    torch.cuda.synchronize()
    for (a, b), (c, d) in zip(imm, dfr):
        assert torch.equal(a, c) and _eq(b, d)


def test_same_weights_twice_flushes_between(gpu):
    """Two deferred calls adding into one dweight: the second queues only
    after flushing the first, so the result is two immediate calls'."""
    import torch
    print("deferred weight finish: same weights twice", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261212)
    for make in (CASES["pw"], CASES["dw_k7"]):
        run, wshape, bsize = make(gpu, gen)
        dw0, db0 = _grads(wshape, bsize, 5)
        dwi, dbi = dw0.clone(), db0.clone()
        run(False, dwi, dbi)
        run(False, dwi, dbi)
        dwd, dbd = dw0.clone(), db0.clone()
        ws1 = run(True, dwd, dbd)
        n1 = gpu.weight_grad_pending()
        ws2 = run(True, dwd, dbd)
        assert gpu.weight_grad_pending() == n1  # the first call's entries flushed
        gpu.weight_grad_flush()
        torch.cuda.synchronize()
        assert torch.equal(dwd, dwi) and torch.equal(dbd, dbi)
        del ws1, ws2


def test_discard_drops_pending_finishes(gpu):
    """A backward pass abandoned part way (its workspace freed) drops its
    pending finishes: they never run, and the next call on the same weights
    does not run them either."""
    import torch
    print("deferred weight finish: discard", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261215)
    run, wshape, bsize = CASES["dw_k7"](gpu, gen)
    dw0, db0 = _grads(wshape, bsize, 9)
    dwi, dbi = dw0.clone(), db0.clone()
    run(False, dwi, dbi)
    dwd, dbd = dw0.clone(), db0.clone()
    _, ws = run(True, dwd, dbd)
    assert gpu.weight_grad_pending() >= 1
    gpu.weight_grad_discard()
    assert gpu.weight_grad_pending() == 0
    del ws  # the abandoned pass's workspace goes away
    torch.cuda.synchronize()
    assert torch.equal(dwd, dw0) and torch.equal(dbd, db0)
    run(False, dwd, dbd)  # into the same weights: only this call adds
    torch.cuda.synchronize()
    assert torch.equal(dwd, dwi) and torch.equal(dbd, dbi)


def test_flush_on_another_stream_is_refused(gpu):
    import torch
    print("deferred weight finish: flush on another stream", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261213)
    run, wshape, bsize = CASES["pw"](gpu, gen)
    dw, db = _grads(wshape, bsize, 3)
    dwi, dbi = dw.clone(), db.clone()
    run(False, dwi, dbi)
    _, ws = run(True, dw, db)
    other = torch.cuda.Stream()
    with pytest.raises(gpu.SoarError):
        gpu.weight_grad_flush(stream=other)
    assert "another stream" in gpu.last_error()
    assert gpu.weight_grad_pending() >= 1
    gpu.weight_grad_flush()
    torch.cuda.synchronize()
    assert torch.equal(dw, dwi) and torch.equal(db, dbi)
    del ws


def test_captured_graph_replays(gpu):
    """Deferred pointwise and depthwise backward calls and the flush
    captured into one graph; every replay, with eager work and
    synchronizations between them, adds what the same calls add eagerly."""
    import torch
    print("deferred weight finish: graph capture", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20261214)
    pw_run, pw_ws, pw_bs = CASES["pw"](gpu, gen)
    dw_run, dw_ws, dw_bs = CASES["dw_k7"](gpu, gen)
    pdw, pdb = _grads(pw_ws, pw_bs, 11)
    ddw, ddb = _grads(dw_ws, dw_bs, 12)
    eager = [t.clone() for t in (pdw, pdb, ddw, ddb)]
    # workspaces allocated before the capture, reused by every replay (each
    # replay's flush has read them before the next replay writes them)
    wpw = _ws(gpu.pw_conv_backward_workspace_bytes(2, 24, 40, 96 * 96))
    wdw = _ws(gpu.lib().soar_dw_conv_backward_workspace_bytes(2, 16, 70, 66, 70, 66, 7, 1, 1))
    # warm-up outside the capture (sets the library up on the device)
    pw_run(False, torch.zeros_like(pdw), torch.zeros_like(pdb), ws=wpw)
    dw_run(False, torch.zeros_like(ddw), torch.zeros_like(ddb), ws=wdw)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        pw_run(True, pdw, pdb, ws=wpw)
        dw_run(True, ddw, ddb, ws=wdw)
        gpu.weight_grad_flush(stream=s)
    assert gpu.weight_grad_pending() == 0
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        pw_run(False, eager[0], eager[1])
        dw_run(False, eager[2], eager[3])
        torch.cuda.synchronize()
        _ = torch.randn(1 << 20, device="cuda").sum().item()  # unrelated eager work
        for got, want in zip((pdw, pdb, ddw, ddb), eager):
            assert torch.equal(got, want), f"replay {rep}"
    np.testing.assert_array_equal(pdw.cpu().numpy(), eager[0].cpu().numpy())
