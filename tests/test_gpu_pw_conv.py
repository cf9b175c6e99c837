"""Parity of the pointwise convolution and the fused CBA forward
(conv -> GroupNorm -> SiLU with the statistics in the conv epilogue) against
the oracle, through the C-ABI of libsoar_gn.so.

Bars (written here, used by every check):
  z (fp32 GEMM, K = C_in terms): |z - z64| <= (C_in + 2) * 2^-24 * (|W| |x| + |b|)
      (the fp32 bound of a K-term dot product, whatever the summation order)
  stats of GroupNorm(z):  as tests/test_gpu_parity.py, 1e-5 relative
  y:                      |d| <= 1e-4 * (1 + |truth|)
The GroupNorm truth is computed by the oracle from the device's own z, so
the GroupNorm bars are not loosened by the convolution's rounding.
"""
import numpy as np
import pytest

from test_gpu_parity import EPS, assert_stats, assert_vals, dev, host

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


@pytest.fixture(params=["default", "mfma", "mfma_no_splitk"])
def pw_path(request, gpu):
    """Runs a test with the default choice between the SIMT and the MFMA
    kernels, with the MFMA kernels forced (SOAR_TUNE_PW_SMALL = 0; small
    grids then split K over blocks where a workspace holds the slices, and
    over the waves of a block), and with the MFMA kernels forced and K split
    only inside blocks (SOAR_TUNE_PW_SPLITK = 1)."""
    old = gpu.tune_get(gpu.TUNE_PW_SMALL)
    old_kz = gpu.tune_get(gpu.TUNE_PW_SPLITK)
    if request.param != "default":
        gpu.tune(gpu.TUNE_PW_SMALL, 0)
    if request.param == "mfma_no_splitk":
        gpu.tune(gpu.TUNE_PW_SPLITK, 1)
    yield request.param
    gpu.tune(gpu.TUNE_PW_SMALL, old)
    gpu.tune(gpu.TUNE_PW_SPLITK, old_kz)


def rng_inputs(seed, N, C_in, C_out, HW, bias=True, kind="normal"):
    r = np.random.default_rng(seed)
    if kind == "offset":
        x = (1e3 + 1e-2 * r.standard_normal((N, C_in, HW))).astype(np.float32)
    else:
        x = r.standard_normal((N, C_in, HW)).astype(np.float32)
    w = (r.uniform(-1.0, 1.0, (C_out, C_in)) / np.sqrt(C_in)).astype(np.float32)
    b = r.uniform(-0.5, 0.5, C_out).astype(np.float32) if bias else None
    return x, w, b


def z_bound(x, w, b, C_in):
    mag = np.einsum("oc,ncp->nop", np.abs(w).astype(np.float64), np.abs(x).astype(np.float64))
    if b is not None:
        mag += np.abs(b).astype(np.float64)[None, :, None]
    return (C_in + 2) * U32 * mag


def assert_z(z, x, w, b, oracle, what=""):
    N, C_in, HW = x.shape
    C_out = w.shape[0]
    truth = oracle.conv1x1_fwd_f64(x, w, b, N, C_in, C_out, HW).reshape(N, C_out, HW)
    err = np.abs(np.asarray(z, np.float64).reshape(N, C_out, HW) - truth)
    bound = z_bound(x, w, b, C_in) + 1e-30
    ratio = err / bound
    i = np.unravel_index(int(np.argmax(ratio)), ratio.shape)
    assert ratio[i] <= 1.0, f"{what} z err {err[i]:.3e} > bound {bound[i]:.3e} at {i}"


CONV_SHAPES = [
    # (C_in, C_out, HW, bias)
    (64, 64, 4096, False),    # fast path, one full 64-row tile
    (64, 64, 4096, True),
    (16, 32, 1000, True),     # fast, partial row tile, ragged item
    (24, 40, 4100, True),     # fast, odd number of K steps (3), partial tile
    (8, 64, 128, False),      # a single K step
    (64, 128, 2048, False),   # two row tiles
    (128, 64, 3000, True),
    (3, 5, 17, True),         # general path: C_in % 8, HW % 4
    (72, 300, 515, True),     # general, five row tiles (two row groups)
    (40, 24, 1, True),        # one pixel
]


@pytest.mark.parametrize("C_in,C_out,HW,bias", CONV_SHAPES)
def test_conv1x1_matches_oracle(gpu, oracle, pw_path, C_in, C_out, HW, bias):
    print(f"conv1x1 C_in={C_in} C_out={C_out} HW={HW} bias={bias}", flush=True)
    x, w, b = rng_inputs(C_in * 7 + HW, 1, C_in, C_out, HW, bias)
    out = gpu.conv1x1_forward(dev(x[0]), dev(w), dev(b) if bias else None)
    assert tuple(out.shape) == (C_out, HW)
    assert_z(host(out)[None], x, w, b, oracle, f"C_in={C_in} C_out={C_out} HW={HW}")


def test_conv1x1_per_sample_loop(gpu, oracle):
    x, w, b = rng_inputs(5, 3, 16, 24, 777)
    out = gpu.conv1x1_forward(dev(x).reshape(3, 16, 777, 1), dev(w), dev(b))
    assert tuple(out.shape) == (3, 24, 777, 1)
    assert_z(host(out), x, w, b, oracle, "N=3")


FUSED_SHAPES = [
    # (N, C_in, C_out, HW, G, kind, silu)
    (1, 64, 64, 4096, 16, "normal", True),
    (2, 32, 48, 2500, 12, "normal", True),     # partial tile, ragged last chunk
    (1, 16, 24, 1030, 6, "normal", False),     # no activation (CBA act=False)
    (1, 8, 16, 17, 4, "normal", True),         # general path
    (1, 64, 64, 70000, 16, "offset", True),    # |mean| / std ~ 1e5
    (1, 130, 72, 4096, 8, "normal", True),     # general path, two row tiles
    (3, 16, 32, 1024, 8, "normal", True),      # exactly one chunk per plane
    # 300 pixel chunks of 1024: the streamed kernel's grid ends in a part-
    # filled window of the XCD-aware block order
    (1, 64, 64, 300 * 1024, 16, "normal", True),
    # small grids with K >= 128: K split over blocks (slices + reduce)
    (1, 256, 128, 4096, 16, "normal", True),   # the Nano LKR at 1024^2, stride 16
    (1, 512, 256, 1024, 32, "offset", True),   # stride 32; large |mean|
    (1, 300, 72, 1000, 8, "normal", False),    # general path (C_in % 8), ragged HW
]


def fused_case(gpu, oracle, N, C_in, C_out, HW, G, kind, silu, seed=3):
    x, w, b = rng_inputs(seed + HW, N, C_in, C_out, HW, True, kind)
    r = np.random.default_rng(seed)
    gamma = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    beta = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    z, y, st = gpu.pw_conv_gn_silu_forward(dev(x), dev(w), dev(b), dev(gamma), dev(beta), G,
                                           eps=EPS, silu=silu)
    return x, w, b, gamma, beta, z, y, st


@pytest.mark.parametrize("N,C_in,C_out,HW,G,kind,silu", FUSED_SHAPES)
def test_pw_conv_gn_silu_matches_oracle(gpu, oracle, pw_path, N, C_in, C_out, HW, G, kind,
                                        silu):
    print(f"pw_conv_gn N={N} C_in={C_in} C_out={C_out} HW={HW} G={G} {kind}", flush=True)
    x, w, b, gamma, beta, z, y, st = fused_case(gpu, oracle, N, C_in, C_out, HW, G, kind,
                                                silu)
    zh = host(z)
    assert_z(zh, x, w, b, oracle, "fused")
    y_t, mean_t, rstd_t = oracle.gn_silu_fwd_f64(zh, gamma, beta, N, C_out, HW, G, EPS,
                                                 silu=silu)
    assert_stats(host(st.mean), host(st.rstd), mean_t, rstd_t, "fused")
    assert_vals(host(y), y_t, "fused y")
    # the saved statistics drive the existing backward: mean + mean_lo is
    # the float64 mean to far below fp32 resolution
    full = host(st.mean).astype(np.float64) + host(st.mean_lo)
    sd = 1.0 / rstd_t
    assert np.all(np.abs(full - mean_t) <= 1e-6 * sd + 1e-9 * np.abs(mean_t))


@pytest.mark.parametrize("N,C_in,C_out,HW,G,kind,silu", FUSED_SHAPES[:3])
def test_pw_conv_gn_matches_unfused_device_path(gpu, oracle, pw_path, N, C_in, C_out, HW, G,
                                                kind, silu):
    """conv (reference signature) then soar_gn_silu_forward on the same z."""
    x, w, b, gamma, beta, z, y, st = fused_case(gpu, oracle, N, C_in, C_out, HW, G, kind,
                                                silu)
    z2 = gpu.conv1x1_forward(dev(x).reshape(N, C_in, HW, 1), dev(w), dev(b)).reshape(z.shape)
    assert np.array_equal(host(z), host(z2))  # same kernel, same operation order
    y2, st2 = gpu.gn_silu_forward(z2, dev(gamma), dev(beta), G, eps=EPS, silu=silu)
    assert_stats(host(st.mean), host(st.rstd), host(st2.mean).astype(np.float64),
                 host(st2.rstd).astype(np.float64), "fused vs unfused")
    assert_vals(host(y), host(y2), "fused vs unfused y")


@pytest.mark.parametrize("N,C_in,C_out,HW,G,silu", [
    (1, 64, 64, 16384, 8, False),   # the LKR block's pw2: epilogue statistics, folded apply
    (2, 32, 48, 70000, 12, True),   # multi-pass apply, SiLU
    (1, 64, 128, 64, 16, False),    # small planes: SIMT conv, one-launch GroupNorm, then an add
    (1, 32, 16, 16384, 2, False),   # small planes: SIMT conv, two-pass GroupNorm
])
def test_pw_conv_gn_add_forward(gpu, oracle, N, C_in, C_out, HW, G, silu):
    """soar_pw_conv_gn_silu_add_forward: y = the CBA forward + residual, bit
    for bit the forward followed by the add (z and the statistics
    unchanged), on every GroupNorm path."""
    import torch
    print(f"pw_conv_gn_add N={N} C_in={C_in} C_out={C_out} HW={HW} G={G} silu={silu}",
          flush=True)
    x, w, b = rng_inputs(HW + C_in + 7, N, C_in, C_out, HW, True)
    r = np.random.default_rng(HW + 3)
    gamma = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    beta = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    res = dev(r.standard_normal((N, C_out, HW)).astype(np.float32))
    args = (dev(x), dev(w), dev(b), dev(gamma), dev(beta), G)
    z0, y0, st0 = gpu.pw_conv_gn_silu_forward(*args, eps=EPS, silu=silu)
    z1, y1, st1 = gpu.pw_conv_gn_silu_forward(*args, eps=EPS, silu=silu, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(z0, z1) and torch.equal(st0.mean, st1.mean)
    assert torch.equal(st0.rstd, st1.rstd) and torch.equal(st0.mean_lo, st1.mean_lo)
    assert torch.equal(y1, y0 + res)


FOLD_SHAPES = [
    # (N, C_in, C_out, HW, G, kind, silu): units past the one-launch size,
    # 256 to 2504 chunk partials each
    (1, 256, 128, 4096, 16, "normal", True),   # the Nano LKR at 1024^2, stride 16: 256
    (1, 128, 256, 4096, 8, "normal", True),    # 1024 partials
    (1, 64, 64, 70000, 16, "offset", True),    # |mean| / std ~ 1e5, ragged: 2188
    (2, 16, 32, 40000, 4, "normal", False),    # two samples, no activation: 2504
]


@pytest.mark.parametrize("N,C_in,C_out,HW,G,kind,silu", FOLD_SHAPES)
def test_pw_conv_gn_folded_finish(gpu, oracle, N, C_in, C_out, HW, G, kind, silu):
    """The finish of the epilogue's chunk partials folded into the apply
    (SOAR_TUNE_FOLD_MAX at or above the unit's partials): no finish launch,
    and z, mean, rstd, mean_lo and y bit for bit those of the separate
    finish (0)."""
    import soar_gn
    import torch
    print(f"pw_conv_gn folded N={N} C_in={C_in} C_out={C_out} HW={HW} G={G} {kind}",
          flush=True)
    old = gpu.tune_get(gpu.TUNE_FOLD_MAX)
    runs = {}
    try:
        for fold in (0, 4096):
            gpu.tune(gpu.TUNE_FOLD_MAX, fold)
            gpu.prof_summary()
            gpu.prof_enable(True)
            try:
                _, _, _, gamma, beta, z, y, st = fused_case(gpu, oracle, N, C_in, C_out, HW,
                                                            G, kind, silu)
                torch.cuda.synchronize()
                names = {r["kernel"] for r in soar_gn.prof_summary()}
            finally:
                gpu.prof_enable(False)
            assert ("gn_stats_finish" in names) == (fold == 0), names
            runs[fold] = [host(t) for t in (z, y, st.mean, st.rstd, st.mean_lo)]
    finally:
        gpu.tune(gpu.TUNE_FOLD_MAX, old)
    for a, b in zip(runs[0], runs[4096]):
        assert np.array_equal(a, b)
    y_t, mean_t, rstd_t = oracle.gn_silu_fwd_f64(runs[4096][0], gamma, beta, N, C_out, HW, G,
                                                 EPS, silu=silu)
    assert_stats(runs[4096][2], runs[4096][3], mean_t, rstd_t, "folded")
    assert_vals(runs[4096][1], y_t, "folded y")


@pytest.mark.parametrize("chunk", [128, 512, 4096])
def test_pw_chunk_changes_only_partial_order(gpu, oracle, chunk):
    args = (1, 32, 32, 10000, 8, "normal", True)
    _, _, _, _, _, z0, y0, st0 = fused_case(gpu, oracle, *args)
    old = gpu.tune_get(gpu.TUNE_PW_CHUNK)
    try:
        gpu.tune(gpu.TUNE_PW_CHUNK, chunk)
        _, _, _, _, _, z1, y1, st1 = fused_case(gpu, oracle, *args)
    finally:
        gpu.tune(gpu.TUNE_PW_CHUNK, old)
    assert np.array_equal(host(z0), host(z1))
    assert_stats(host(st1.mean), host(st1.rstd), host(st0.mean).astype(np.float64),
                 host(st0.rstd).astype(np.float64), f"chunk {chunk}")
    assert_vals(host(y1), host(y0), f"chunk {chunk} y")


def test_pw_conv_full_size_cba(gpu):
    """CBA pointwise conv at config 3's GroupNorm shape: 64 -> 64 channels at
    2048x2048, G = 16.  z is spot-checked against float64 on 4096 random
    pixel columns; statistics and y against the unfused device path (which
    test_gpu_parity.py pins to the oracle at this size)."""
    import torch
    C, HW, G = 64, 2048 * 2048, 16
    print("pw_conv full size 64->64 2048^2", flush=True)
    x = torch.empty((1, C, 2048, 2048), dtype=torch.float32, device="cuda")
    gpu.synth_normal(x, 1234, 1)
    r = np.random.default_rng(9)
    w = (r.uniform(-1, 1, (C, C)) / 8.0).astype(np.float32)
    gamma = r.uniform(0.5, 1.5, C).astype(np.float32)
    beta = (0.1 * r.standard_normal(C)).astype(np.float32)
    z, y, st = gpu.pw_conv_gn_silu_forward(x, dev(w), None, dev(gamma), dev(beta), G, eps=EPS)
    torch.cuda.synchronize()
    cols = torch.from_numpy(np.sort(r.choice(HW, 4096, replace=False))).cuda()
    xs = host(x.reshape(C, HW).index_select(1, cols)).astype(np.float64)
    zs = host(z.reshape(C, HW).index_select(1, cols)).astype(np.float64)
    truth = w.astype(np.float64) @ xs
    bound = (C + 2) * U32 * (np.abs(w).astype(np.float64) @ np.abs(xs))
    assert np.all(np.abs(zs - truth) <= bound)
    y2, st2 = gpu.gn_silu_forward(z, dev(gamma), dev(beta), G, eps=EPS)
    assert_stats(host(st.mean), host(st.rstd), host(st2.mean).astype(np.float64),
                 host(st2.rstd).astype(np.float64), "full size")
    d = (y - y2).abs().max().item()
    assert d <= 1e-4 * (1.0 + y2.abs().max().item()), d
    del x, z, y, y2


def test_pw_conv_errors(gpu):
    import ctypes
    import torch
    L = gpu.lib()
    x = torch.zeros((1, 8, 16), device="cuda")
    w = torch.zeros((16, 8), device="cuda")
    out = torch.zeros((16, 16), device="cuda")
    rc = L.soar_conv2d_1x1_forward(None, ctypes.c_void_p(w.data_ptr()), None,
                                   ctypes.c_void_p(out.data_ptr()), 8, 16, 16, None)
    assert rc == gpu.SOAR_EINVAL and "NULL" in gpu.last_error()
    hostbuf = np.zeros(8 * 16, np.float32)
    rc = L.soar_conv2d_1x1_forward(ctypes.c_void_p(hostbuf.ctypes.data),
                                   ctypes.c_void_p(w.data_ptr()), None,
                                   ctypes.c_void_p(out.data_ptr()), 8, 16, 16, None)
    assert rc == gpu.SOAR_EINVAL and "not device memory" in gpu.last_error()
    # an output whose allocation ends before the shape does (the arena gives
    # an allocation whose end is known exactly): 16 x 16 floats do not fit
    # in the last 512 bytes
    arena = ctypes.c_void_p()
    gpu.check(L.soar_arena_create(1 << 20, 256, ctypes.byref(arena)))
    try:
        p = ctypes.c_void_p()
        gpu.check(L.soar_arena_alloc(arena, (1 << 20) - 512, ctypes.byref(p), None))
        gpu.check(L.soar_arena_alloc(arena, 512, ctypes.byref(p), None))
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = L.soar_conv2d_1x1_forward(ctypes.c_void_p(x.data_ptr()),
                                       ctypes.c_void_p(w.data_ptr()), None, p, 8, 16, 16, s)
        assert rc == gpu.SOAR_EINVAL and "allocation holds" in gpu.last_error()
        rc = L.soar_conv2d_1x1_forward(ctypes.c_void_p(x.data_ptr()),
                                       ctypes.c_void_p(w.data_ptr()), None, p, 8, 8, 16, s)
        assert rc == gpu.SOAR_OK  # 8 x 16 floats fit exactly
        torch.cuda.synchronize()
    finally:
        gpu.check(L.soar_arena_destroy(arena))


# ---- backward ----------------------------------------------------------------------

def bwd_bounds(dz, x, w):
    """fp32 bounds of dx (C_out-term sums) and of dw, db (pixel sums)."""
    N, C_out, HW = dz.shape
    C_in = x.shape[1]
    ad, ax, aw = (np.abs(a).astype(np.float64) for a in (dz, x, w))
    bx = (C_out + 2) * U32 * np.einsum("oc,nop->ncp", aw, ad)
    mw = np.einsum("nop,ncp->oc", ad, ax)
    mb = ad.sum(axis=(0, 2))
    K = N * HW + 2
    return bx, K * U32 * mw, K * U32 * mb


BWD_SHAPES = [
    # (N, C_in, C_out, HW)
    (1, 64, 64, 4096),
    (2, 32, 48, 2500),      # partial dW tiles, ragged chunks
    (1, 16, 24, 1030),
    (1, 8, 16, 17),         # general paths (HW % 4)
    (1, 64, 128, 2048),     # two row tiles of dW / dx
    (1, 130, 72, 4096),     # C_in % 8 != 0 for the forward; dx K = 72
    (3, 24, 8, 333),
    (1, 128, 256, 4096),    # dx: K = 256 over the waves of a block (small grid)
    (1, 72, 200, 1000),     # dx: general path, small grid
]


@pytest.mark.parametrize("N,C_in,C_out,HW", BWD_SHAPES)
def test_pw_conv_backward_matches_oracle(gpu, oracle, pw_path, N, C_in, C_out, HW):
    print(f"pw_conv_backward N={N} C_in={C_in} C_out={C_out} HW={HW}", flush=True)
    r = np.random.default_rng(N * 1000 + C_in + HW)
    dz = r.standard_normal((N, C_out, HW)).astype(np.float32)
    x = r.standard_normal((N, C_in, HW)).astype(np.float32)
    w = (r.uniform(-1, 1, (C_out, C_in)) / np.sqrt(C_in)).astype(np.float32)
    dx, dw, db = gpu.pw_conv_backward(dev(dz), dev(x), dev(w))
    tx, tw, tb = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    bx, bw, bb = bwd_bounds(dz, x, w)
    for got, t, b, name in ((dx, tx, bx, "dx"), (dw, tw, bw, "dw"), (db, tb, bb, "db")):
        err = np.abs(host(got).astype(np.float64).reshape(-1) - t)
        ratio = err / (b.reshape(-1) + 1e-30)
        i = int(np.argmax(ratio))
        assert ratio[i] <= 1.0, f"{name} err {err[i]:.3e} > bound {b.reshape(-1)[i]:.3e} at {i}"


WGRAD_WAVE_SHAPES = [
    # (N, C_in, C_out, HW)
    (1, 64, 64, 65536),     # one 64 x 64 tile, 1024 wave chunks of 64 pixels
    (3, 24, 8, 333),        # one block per plane: 11 steps over up to 8 waves
    (1, 130, 72, 4096),     # 6 partial tiles, ragged rows and columns
    (2, 32, 48, 2500),      # 32-column tiles; the last block of a plane is short
]


@pytest.mark.parametrize("N,C_in,C_out,HW", WGRAD_WAVE_SHAPES)
def test_pw_wgrad_waves_per_block(gpu, oracle, restore_pw_small, N, C_in, C_out, HW):
    """The MFMA weight gradient with 1, 2, 4 and 8 waves per block (the
    waves of a block take interleaved steps of one chunk and add their
    tiles in LDS before writing one partial):
    every setting within the fp32 bound of the float64 oracle, and each
    one bitwise repeatable."""
    print(f"pw wgrad waves N={N} C_in={C_in} C_out={C_out} HW={HW}", flush=True)
    old = gpu.tune_get(gpu.TUNE_PW_WG_WAVES)
    gpu.tune(gpu.TUNE_PW_SMALL, 0)
    r = np.random.default_rng(HW + C_in)
    dz = r.standard_normal((N, C_out, HW)).astype(np.float32)
    x = r.standard_normal((N, C_in, HW)).astype(np.float32)
    w = (r.uniform(-1, 1, (C_out, C_in)) / np.sqrt(C_in)).astype(np.float32)
    _, tw, tb = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    _, bw, bb = bwd_bounds(dz, x, w)
    dzd, xd, wd = dev(dz), dev(x), dev(w)
    try:
        for waves in (1, 2, 4, 8):
            gpu.tune(gpu.TUNE_PW_WG_WAVES, waves)
            runs = []
            for _ in range(2):
                _, dw, db = gpu.pw_conv_backward(dzd, xd, wd, want_dx=False)
                runs.append((host(dw), host(db)))
            for got, t, bnd, name in ((runs[0][0], tw, bw, "dw"), (runs[0][1], tb, bb, "db")):
                err = np.abs(got.astype(np.float64).reshape(-1) - t)
                ratio = err / (bnd.reshape(-1) + 1e-30)
                i = int(np.argmax(ratio))
                assert ratio[i] <= 1.0, f"waves {waves} {name} err {err[i]:.3e} at {i}"
            assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1])
    finally:
        gpu.tune(gpu.TUNE_PW_WG_WAVES, old)


@pytest.mark.parametrize("C_in,C_out,HW", [(32, 32, 1000), (128, 256, 2048)])
def test_pw_conv_backward_accumulates(gpu, oracle, pw_path, C_in, C_out, HW):
    N = 1
    r = np.random.default_rng(4)
    dz = r.standard_normal((N, C_out, HW)).astype(np.float32)
    x = r.standard_normal((N, C_in, HW)).astype(np.float32)
    w = r.uniform(-0.2, 0.2, (C_out, C_in)).astype(np.float32)
    dx0 = r.standard_normal((N, C_in, HW)).astype(np.float32)
    dw0 = r.standard_normal((C_out, C_in)).astype(np.float32)
    db0 = r.standard_normal(C_out).astype(np.float32)
    dx, dw, db = gpu.pw_conv_backward(dev(dz), dev(x), dev(w), dx=dev(dx0), dweight=dev(dw0),
                                      dbias=dev(db0), accumulate_dx=True)
    tx, tw, tb = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    bx, bw, bb = bwd_bounds(dz, x, w)
    assert np.all(np.abs(host(dx).reshape(-1) - (dx0.reshape(-1) + tx)) <=
                  bx.reshape(-1) + U32 * np.abs(dx0).reshape(-1) * 2)
    assert np.all(np.abs(host(dw).reshape(-1) - (dw0.reshape(-1) + tw)) <=
                  bw.reshape(-1) + U32 * np.abs(dw0).reshape(-1) * 2 + 1e-30)
    assert np.all(np.abs(host(db) - (db0 + tb)) <= bb + U32 * np.abs(db0) * 2 + 1e-30)
    # only some gradients
    dx2, dw2, db2 = gpu.pw_conv_backward(dev(dz), dev(x), dev(w), want_dx=False, want_db=False)
    assert dx2 is None and db2 is None
    assert np.all(np.abs(host(dw2).reshape(-1) - tw) <= bw.reshape(-1) + 1e-30)


def test_conv2d_1x1_backward_reference_signature(gpu, oracle):
    """grad_in/grad_weight/grad_bias += as the reference kernels, one sample."""
    import ctypes
    import torch
    C_in, C_out, HW = 24, 40, 1500
    r = np.random.default_rng(5)
    go = r.standard_normal((C_out, HW)).astype(np.float32)
    x = r.standard_normal((C_in, HW)).astype(np.float32)
    w = r.uniform(-0.3, 0.3, (C_out, C_in)).astype(np.float32)
    gi0 = r.standard_normal((C_in, HW)).astype(np.float32)
    gi, gw, gb = dev(gi0), torch.zeros((C_out, C_in), device="cuda"), torch.zeros(C_out,
                                                                                 device="cuda")
    go_d, x_d, w_d = dev(go), dev(x), dev(w)  # kept alive across the calls
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    gpu.check(gpu.lib().soar_conv2d_1x1_backward(P(go_d), P(x_d), P(w_d), P(gi), P(gw),
                                                 P(gb), C_in, C_out, HW, None))
    torch.cuda.synchronize()
    ri, rw, rb = oracle.ref_conv1x1_bwd_f32(go, x, w, C_in, C_out, HW, grad_in=gi0.copy())
    tx, tw, tb = oracle.conv1x1_bwd_f64(go[None], x[None], w, 1, C_in, C_out, HW)
    bx, bw, bb = bwd_bounds(go[None], x[None], w)
    assert np.all(np.abs(host(gi).reshape(-1) - (gi0.reshape(-1) + tx)) <=
                  bx.reshape(-1) + 2 * U32 * np.abs(gi0).reshape(-1))
    assert np.all(np.abs(host(gw).reshape(-1) - tw) <= bw.reshape(-1) + 1e-30)
    assert np.all(np.abs(host(gb) - tb) <= bb + 1e-30)
    # and the reference's own fp32 loops agree within the same bounds
    assert np.all(np.abs(rw - tw) <= bw.reshape(-1) + 1e-30)
    # NULL outputs are skipped
    gpu.check(gpu.lib().soar_conv2d_1x1_backward(P(go_d), P(x_d), P(w_d), None, None,
                                                 P(gb), C_in, C_out, HW, None))
    torch.cuda.synchronize()
    assert np.all(np.abs(host(gb) - 2 * tb) <= 2 * bb + 1e-30)


def test_pw_conv_backward_full_size_adjoint(gpu):
    """64 -> 64 at 2048x2048: dx on 4096 random pixel columns against float64,
    and the adjoint identities <W, dW> = <z, dz> = <x, dx> (z = W x) that
    tie dW and dx to the forward at full size."""
    import torch
    C, HW = 64, 2048 * 2048
    print("pw_conv_backward full size", flush=True)
    x = torch.empty((1, C, HW), device="cuda")
    dz = torch.empty((1, C, HW), device="cuda")
    gpu.synth_normal(x, 77, 1)
    gpu.synth_normal(dz, 77, 4)
    r = np.random.default_rng(10)
    w = dev((r.uniform(-1, 1, (C, C)) / 8.0).astype(np.float32))
    dx, dw, db = gpu.pw_conv_backward(dz, x, w)
    z = gpu.conv1x1_forward(x.reshape(1, C, HW, 1), w).reshape(1, C, HW)
    torch.cuda.synchronize()
    zdz = torch.dot(z.reshape(-1).double(), dz.reshape(-1).double()).item()
    wdw = torch.dot(w.reshape(-1).double(), dw.reshape(-1).double()).item()
    xdx = torch.dot(x.reshape(-1).double(), dx.reshape(-1).double()).item()
    scale = torch.dot(z.reshape(-1).double().abs(), dz.reshape(-1).double().abs()).item()
    assert abs(wdw - zdz) <= 1e-5 * scale, (wdw, zdz, scale)
    assert abs(xdx - zdz) <= 1e-5 * scale, (xdx, zdz, scale)
    assert abs(db.double().sum().item() - dz.double().sum().item()) <= 1e-5 * (
        dz.double().abs().sum().item())
    cols = torch.from_numpy(np.sort(r.choice(HW, 4096, replace=False))).cuda()
    ds = host(dz.reshape(C, HW).index_select(1, cols)).astype(np.float64)
    xs = host(dx.reshape(C, HW).index_select(1, cols)).astype(np.float64)
    wh = host(w).astype(np.float64)
    bound = (C + 2) * U32 * (np.abs(wh).T @ np.abs(ds))
    assert np.all(np.abs(xs - wh.T @ ds) <= bound)
    del x, dz, dx, z


# ---- small convolutions: the SIMT kernels (SOAR_TUNE_PW_SMALL) ---------------------

SMALL_PW_SHAPES = [
    # (N, C_in, C_out, HW, bias)
    (1, 256, 512, 4, True),    # SOAR Nano stride-32 pointwise convs at a 64x64 image
    (1, 128, 256, 16, False),  # stride 16
    (2, 64, 128, 64, True),
    (1, 32, 64, 256, True),
    (1, 64, 128, 2048, True),  # 2^24 multiply-adds: SIMT by default
    (3, 5, 7, 9, True),        # C_in % 4 != 0: scalar weight loads; rows straddle waves
    (1, 600, 40, 3, True),     # K split over 15 waves of 40 channels
    (4, 24, 8, 1, False),      # one pixel
    (2, 1, 3, 5, True),        # K = 1
    (3, 16, 24, 100, True),    # weight-gradient segments cross sample planes
    # few input channels over many pixels: a thread per pixel (k_pw_px)
    (1, 16, 16, 65536, True),  # SOAR Nano Fuse at 1024^2 (256^2 planes); dx K = 16 too
    (2, 32, 8, 4096, False),   # K = 32, two samples; dx K = 8
    (1, 8, 40, 1030, True),    # three output tiles, ragged pixel blocks; dx K = 40: per output
    (1, 16, 4, 262144, False), # the Nano head's prediction at 512^2: dx K = 4
    (1, 64, 8, 65536, True),   # K = 64 over 65536 pixels; dx K = 8
]


@pytest.fixture
def restore_pw_small(gpu):
    old = gpu.tune_get(gpu.TUNE_PW_SMALL)
    old_kz = gpu.tune_get(gpu.TUNE_PW_SPLITK)
    yield
    gpu.tune(gpu.TUNE_PW_SMALL, old)
    gpu.tune(gpu.TUNE_PW_SPLITK, old_kz)


def _assert_bwd(got, truth, bounds, what, base=None):
    for g, t, b, name in zip(got, truth, bounds, ("dx", "dw", "db")):
        if g is None:
            continue
        h = host(g).astype(np.float64).reshape(-1)
        lim = b.reshape(-1) + 1e-30
        if base is not None:
            b0 = base[name].astype(np.float64).reshape(-1)
            h = h - b0
            lim = lim + 2 * U32 * np.abs(b0)
        err = np.abs(h - t)
        i = int(np.argmax(err / lim))
        assert err[i] <= lim[i], f"{what} {name} err {err[i]:.3e} > bound {lim[i]:.3e} at {i}"


@pytest.mark.parametrize("N,C_in,C_out,HW,bias", SMALL_PW_SHAPES)
def test_pw_small_planes_match_oracle(gpu, oracle, restore_pw_small, N, C_in, C_out, HW, bias):
    """Forward, fused CBA forward and backward of small convolutions, through
    the SIMT kernels (limit 2^40) and through the MFMA kernels (limit 0),
    with and without K split over blocks, each against the oracle's float64
    results within the fp32 bounds above."""
    print(f"pw small N={N} C_in={C_in} C_out={C_out} HW={HW}", flush=True)
    x, w, b = rng_inputs(N * 31 + C_in + HW, N, C_in, C_out, HW, bias)
    r = np.random.default_rng(HW + C_out)
    dz = r.standard_normal((N, C_out, HW)).astype(np.float32)
    gamma = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    beta = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    G = 2 if C_out % 2 == 0 else 1
    bd = dev(b) if bias else None
    truth_b = oracle.conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW)
    bounds = bwd_bounds(dz, x, w)
    for lim, kz in ((1 << 40, 8), (0, 8), (0, 1)):
        gpu.tune(gpu.TUNE_PW_SMALL, lim)
        gpu.tune(gpu.TUNE_PW_SPLITK, kz)
        what = f"limit {lim} splitk {kz}"
        z = gpu.pw_conv_forward(dev(x), dev(w), bd)
        assert_z(host(z), x, w, b, oracle, what)
        zf, y, st = gpu.pw_conv_gn_silu_forward(dev(x), dev(w), bd, dev(gamma), dev(beta), G,
                                                eps=EPS)
        if lim == 0 and kz > 1:
            # the fused entry may split K over blocks (its workspace holds the
            # slices), the plain entry has no workspace: other summation order
            assert_z(host(zf), x, w, b, oracle, what + " fused")
        else:
            assert np.array_equal(host(zf), host(z)), what  # one kernel behind both entries
        y_t, mean_t, rstd_t = oracle.gn_silu_fwd_f64(host(zf), gamma, beta, N, C_out, HW, G,
                                                     EPS, silu=True)
        assert_stats(host(st.mean), host(st.rstd), mean_t, rstd_t, what)
        assert_vals(host(y), y_t, what + " y")
        got = gpu.pw_conv_backward(dev(dz), dev(x), dev(w))
        _assert_bwd(got, truth_b, bounds, what)
    # the SIMT path's accumulation contract, and each gradient alone
    gpu.tune(gpu.TUNE_PW_SMALL, 1 << 40)
    base = {"dx": r.standard_normal((N, C_in, HW)).astype(np.float32),
            "dw": r.standard_normal((C_out, C_in)).astype(np.float32),
            "db": r.standard_normal(C_out).astype(np.float32)}
    got = gpu.pw_conv_backward(dev(dz), dev(x), dev(w), dx=dev(base["dx"]),
                               dweight=dev(base["dw"]), dbias=dev(base["db"]),
                               accumulate_dx=True)
    _assert_bwd(got, truth_b, bounds, "accumulate", base)
    # dx, dW and db together run as one launch (k_pw_small_bwd): the same
    # bits as each gradient computed alone
    together = [host(t) for t in gpu.pw_conv_backward(dev(dz), dev(x), dev(w))]
    for k, want in enumerate(("dx", "dw", "db")):
        got = gpu.pw_conv_backward(dev(dz), dev(x), dev(w), want_dx=want == "dx",
                                   want_dw=want == "dw", want_db=want == "db")
        _assert_bwd(got, truth_b, bounds, f"only {want}")
        assert sum(g is not None for g in got) == 1
        assert np.array_equal(host(got[k]), together[k]), f"{want} alone vs together"
    z0 = dev(np.full((N, C_out, HW), 0.25, np.float32))
    gpu.pw_conv_forward(dev(x), dev(w), bd, z=z0)
    assert_z(host(z0), x, w, b, oracle, "into a given z")


DETERMINISM_CASES = [
    # (N, C_in, C_out, HW, limit): which path runs
    (1, 256, 512, 16, None),        # SIMT forward / dx / weight gradient (K split over waves)
    (1, 256, 128, 4096, None),      # MFMA small grid: K over 4 blocks x 4 waves, slice reduce
                                    # with the statistics; dx K over the waves of a block
    (1, 64, 64, 262144, None),      # MFMA, two K steps in flight (large grid)
    (3, 24, 40, 1000, 0),           # MFMA forced, general shapes
]


@pytest.mark.parametrize("N,C_in,C_out,HW,limit", DETERMINISM_CASES)
def test_pw_paths_are_deterministic(gpu, oracle, restore_pw_small, N, C_in, C_out, HW, limit):
    """Every pointwise path sums in a fixed order (no atomics): two runs of the
    fused forward and of the backward are bitwise identical."""
    print(f"pw determinism N={N} C_in={C_in} C_out={C_out} HW={HW}", flush=True)
    if limit is not None:
        gpu.tune(gpu.TUNE_PW_SMALL, limit)
    x, w, b = rng_inputs(HW + C_out, N, C_in, C_out, HW)
    r = np.random.default_rng(C_in)
    dz = r.standard_normal((N, C_out, HW)).astype(np.float32)
    gamma = r.uniform(0.5, 1.5, C_out).astype(np.float32)
    beta = (0.1 * r.standard_normal(C_out)).astype(np.float32)
    G = 8 if C_out % 8 == 0 else 4
    xd, wd, bd, dzd = dev(x), dev(w), dev(b), dev(dz)
    runs = []
    for _ in range(2):
        z, y, st = gpu.pw_conv_gn_silu_forward(xd, wd, bd, dev(gamma), dev(beta), G, eps=EPS)
        dx, dw, db = gpu.pw_conv_backward(dzd, xd, wd)
        runs.append([host(t) for t in (z, y, st.mean, st.rstd, dx, dw, db)])
    for a, c in zip(*runs):
        assert np.array_equal(a, c)
