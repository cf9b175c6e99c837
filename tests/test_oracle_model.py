"""Pins of the model-level oracle (oracle/soar_model_ref.py) - CPU.

Each restated piece is checked against something independent of the way
it is written: brute-force loops of the reference's own formulas
(layers.cpp:1100-1150 resize, :975-985 pixel shuffle, soar_model.cpp:
99-122 pad, losses.cpp:101-108,240-249 loss), the C oracle's float64
convolution / GroupNorm statements for the CBA blocks, central finite
differences for the model gradients, a closed form for AdamW's first step,
hand-checked RLE strings, and the .soar byte layout.
"""
import math
import struct

import numpy as np
import pytest
import torch

import soar_model_ref as smr

F32 = np.float32


def rng(seed):
    return np.random.default_rng(seed)


# ---- resize (Upsample) -------------------------------------------------------
def upsample_loop(x, Ho, Wo):
    """layers.cpp:1100-1130, float32 index arithmetic, float64 values."""
    C, H, W = x.shape
    sy, sx = F32(H) / F32(Ho), F32(W) / F32(Wo)
    out = np.zeros((C, Ho, Wo))
    for c in range(C):
        for y in range(Ho):
            for xx in range(Wo):
                fy = max(F32((F32(y) + F32(0.5)) * sy - F32(0.5)), F32(0))
                fx = max(F32((F32(xx) + F32(0.5)) * sx - F32(0.5)), F32(0))
                y0, x0 = int(math.floor(fy)), int(math.floor(fx))
                y1, x1 = min(y0 + 1, H - 1), min(x0 + 1, W - 1)
                y0, x0 = min(y0, H - 1), min(x0, W - 1)
                ly, lx = float(fy) - y0, float(fx) - x0
                hy, hx = 1 - ly, 1 - lx
                out[c, y, xx] = (hy * (hx * x[c, y0, x0] + lx * x[c, y0, x1]) +
                                 ly * (hx * x[c, y1, x0] + lx * x[c, y1, x1]))
    return out


def upsample_bwd_loop(go, H, W):
    """UpsampleNode CPU backward (layers.cpp:1021-1066): the scatter."""
    C, Ho, Wo = go.shape
    sy, sx = F32(H) / F32(Ho), F32(W) / F32(Wo)
    gx = np.zeros((C, H, W))
    for c in range(C):
        for y in range(Ho):
            for xx in range(Wo):
                fy = max(F32((F32(y) + F32(0.5)) * sy - F32(0.5)), F32(0))
                fx = max(F32((F32(xx) + F32(0.5)) * sx - F32(0.5)), F32(0))
                y0, x0 = int(math.floor(fy)), int(math.floor(fx))
                y1, x1 = min(y0 + 1, H - 1), min(x0 + 1, W - 1)
                y0, x0 = min(y0, H - 1), min(x0, W - 1)
                ly, lx = float(fy) - y0, float(fx) - x0
                g = go[c, y, xx]
                gx[c, y0, x0] += (1 - ly) * (1 - lx) * g
                gx[c, y0, x1] += (1 - ly) * lx * g
                gx[c, y1, x0] += ly * (1 - lx) * g
                gx[c, y1, x1] += ly * lx * g
    return gx


@pytest.mark.parametrize("H,W,th", [(2, 2, 4), (4, 4, 16), (3, 5, 6), (4, 6, 8)])
def test_resize_matches_reference_loop(H, W, th):
    x = rng(1).normal(size=(2, H, W))
    t = torch.tensor(x[None], requires_grad=True)
    out = smr.resize_bilinear(t, th, int(round(W * th / H)))
    Ho, Wo = out.shape[2:]
    np.testing.assert_allclose(out.detach().numpy()[0], upsample_loop(x, Ho, Wo),
                               rtol=1e-12, atol=1e-12)
    go = rng(2).normal(size=(2, Ho, Wo))
    out.backward(torch.tensor(go[None]))
    np.testing.assert_allclose(t.grad.numpy()[0], upsample_bwd_loop(go, H, W),
                               rtol=1e-12, atol=1e-12)


def test_pixel_shuffle_matches_reference_index():
    r = 2
    x = rng(3).normal(size=(1, 8, 3, 5))
    out = torch.nn.functional.pixel_shuffle(torch.tensor(x), r).numpy()[0]
    C_out, Ho, Wo = out.shape
    for c in range(C_out):
        for y in range(Ho):
            for xx in range(Wo):
                cin = c * r * r + (y % r) * r + (xx % r)  # layers.cpp:975-985
                assert out[c, y, xx] == x[0, cin, y // r, xx // r]


@pytest.mark.parametrize("H,W,ph,pw", [(5, 7, 3, 1), (4, 4, 4, 2), (2, 3, 30, 29)])
def test_pad_matches_reference_loop(H, W, ph, pw):
    x = rng(4).normal(size=(2, H, W))
    t = torch.tensor(x[None], requires_grad=True)
    out = smr.pad_spatial(t, ph, pw)
    reflect = ph < H and pw < W  # soar_model.cpp:96
    exp = np.zeros((2, H + ph, W + pw))
    src = np.zeros((2, H + ph, W + pw), dtype=np.int64)
    for c in range(2):
        for y in range(H + ph):
            ys = y if y < H else (2 * (H - 1) - y if reflect else H - 1)
            for xx in range(W + pw):
                xs = xx if xx < W else (2 * (W - 1) - xx if reflect else W - 1)
                exp[c, y, xx] = x[c, ys, xs]
                src[c, y, xx] = (c * H + ys) * W + xs
    np.testing.assert_array_equal(out.detach().numpy()[0], exp)
    go = rng(5).normal(size=exp.shape)
    out.backward(torch.tensor(go[None]))
    gi = np.zeros(2 * H * W)
    np.add.at(gi, src.ravel(), go.ravel())  # AutoPadNode (soar_model.cpp:25-34)
    np.testing.assert_allclose(t.grad.numpy()[0].ravel(), gi, rtol=1e-13, atol=1e-13)


# ---- loss --------------------------------------------------------------------
def test_loss_forward_matches_reference_loops():
    n = 257
    z = rng(6).normal(0, 3, size=n)
    y = (rng(7).uniform(size=n) < 0.3).astype(np.float64)
    lo = smr.dice_bce_forward(z, y)
    bce = 0.0
    inter = sp = sy = 0.0
    for zi, yi in zip(z, y):
        w = 1.0 + (3.0 - 1.0) * yi
        bce += (1 - yi) * zi + w * (max(-zi, 0.0) + math.log(1.0 + math.exp(-abs(zi))))
        p = 1.0 / (1.0 + math.exp(-zi))
        inter += p * yi
        sp += p
        sy += yi
    bce /= n
    dice = 1.0 - (2 * inter + 1.0) / (sp + sy + 1.0 + 1e-7)
    assert abs(lo.bce - bce) < 1e-12 and abs(lo.dice - dice) < 1e-12
    assert abs(lo.total - (0.5 * bce + 0.5 * dice)) < 1e-12


def test_loss_backward_formula_is_the_gradient():
    """The reference's backward formula (loss_kernels.cu:212-252) against
    central differences of the forward (equal up to the forward's 1e-7)."""
    n = 64
    z = rng(8).normal(0, 2, size=n)
    y = (rng(9).uniform(size=n) < 0.4).astype(np.float64)
    lo = smr.dice_bce_forward(z, y)
    g = smr.dice_bce_grad(z, y, lo)
    for i in (0, 5, 33, 63):
        h = 1e-6
        zp, zm = z.copy(), z.copy()
        zp[i] += h
        zm[i] -= h
        fd = (smr.dice_bce_forward(zp, y).total - smr.dice_bce_forward(zm, y).total) / (2 * h)
        assert abs(fd - g[i]) <= 1e-6 * max(1e-3, abs(fd)) + 1e-9


# ---- CBA blocks against the C oracle -----------------------------------------
def test_cba_matches_c_oracle(oracle):
    """Model.cba (torch conv2d + group_norm + silu) equals the C oracle's
    float64 convolution and GroupNorm statements for a pointwise and a
    depthwise stride-2 block."""
    r = rng(10)
    C1, C2, H, W = 6, 12, 9, 10
    x = r.normal(size=(C1, H, W)).astype(F32)
    w_pw = r.uniform(-0.4, 0.4, size=(C2, C1, 1, 1)).astype(F32)
    g = r.uniform(0.5, 1.5, size=C2).astype(F32)
    b = r.normal(0, 0.1, size=C2).astype(F32)
    m = smr.Model({"a.conv.weight": w_pw, "a.norm.weight": g, "a.norm.bias": b},
                  requires_grad=False)
    out = m.cba("a", torch.tensor(x[None].astype(np.float64))).numpy()[0]
    z = oracle.conv1x1_fwd_f64(x, w_pw.reshape(C2, C1), None, 1, C1, C2, H * W)
    G = smr.select_group_count(C2)
    y, _, _ = oracle.gn_silu_fwd_f64(z.astype(F32), g, b, 1, C2, H * W, G, smr.GN_EPS)
    # the C oracle reads fp32 inputs: compare against torch on the same fp32 z
    zt = torch.tensor(z.astype(F32).astype(np.float64).reshape(1, C2, H, W))
    ref = torch.nn.functional.silu(torch.nn.functional.group_norm(
        zt, G, torch.tensor(g.astype(np.float64)), torch.tensor(b.astype(np.float64)),
        eps=smr.GN_EPS)).numpy()[0]
    np.testing.assert_allclose(ref.ravel(), y, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(
        m.conv("a.conv", torch.tensor(x[None].astype(np.float64))).numpy().ravel(), z,
        rtol=1e-12, atol=1e-12)
    assert out.shape == (C2, H, W)
    # depthwise k3 stride 2 (Down.dw)
    w_dw = r.uniform(-0.5, 0.5, size=(C1, 1, 3, 3)).astype(F32)
    m2 = smr.Model({"d.conv.weight": w_dw}, requires_grad=False)
    zt = m2.conv("d.conv", torch.tensor(x[None].astype(np.float64)), 3, 2, -1, 1, C1).numpy()
    zd = oracle.dw_fwd_f64(x[None], w_dw, None, 1, C1, H, W, 3, 1, 2, 1)
    np.testing.assert_allclose(zt, zd, rtol=1e-12, atol=1e-12)


def test_general_conv_matches_loop():
    """The stem's grouped convolution (k3, stride 2, groups 1) against a
    direct loop of conv2d_forward's definition."""
    r = rng(11)
    x = r.normal(size=(2, 9, 8))
    w = r.normal(size=(4, 2, 3, 3))
    m = smr.Model({"c.weight": w}, requires_grad=False)
    out = m.conv("c", torch.tensor(x[None]), 3, 2).numpy()[0]
    Ho, Wo = (9 + 2 - 3) // 2 + 1, (8 + 2 - 3) // 2 + 1
    exp = np.zeros((4, Ho, Wo))
    for co in range(4):
        for oy in range(Ho):
            for ox in range(Wo):
                s = 0.0
                for ci in range(2):
                    for ky in range(3):
                        for kx in range(3):
                            iy, ix = oy * 2 - 1 + ky, ox * 2 - 1 + kx
                            if 0 <= iy < 9 and 0 <= ix < 8:
                                s += w[co, ci, ky, kx] * x[ci, iy, ix]
                exp[co, oy, ox] = s
    np.testing.assert_allclose(out, exp, rtol=1e-12, atol=1e-12)


# ---- the model ---------------------------------------------------------------
def test_model_spec_counts():
    """Parameter counts grow with the variant (the reference's own
    assertions, tests/test_full_engine.cpp:19-33) and names follow the
    registration of soar_model.cpp:211-255."""
    counts = [sum(int(np.prod(s)) for _, s, _ in smr.model_spec(1, 1, v)) for v in range(5)]
    assert counts[0] > 200000
    assert counts[0] < counts[1] < counts[2] < counts[3] < counts[4]
    names = [n for n, _, _ in smr.model_spec(1, 1, 0)]
    assert len(names) == len(set(names))
    assert names[0] == "l0_cba.conv.weight" and names[-1] == "l9_ctx.gate_conv.weight"
    for must in ("l6_lkr_0.pw2.norm.weight", "l6_lkr_1.dw.conv.weight", "l2_lkr.dw.conv.weight",
                 "l15_agg.proj_2.norm.bias", "l17_head.pred.bias", "l9_ctx.branch_2.conv.weight"):
        assert must in names
    # map order: a module's own parameters first, then submodules by name
    i = names.index("l17_head.pred.bias")
    assert names[i + 1] == "l17_head.pred.weight"
    assert names.index("l10_fuse.gate_conv.bias") < names.index("l10_fuse.gate_dw.conv.weight")


def test_model_forward_shapes_and_padding():
    spec = smr.model_spec(1, 1, 0)
    w = smr.random_weights(spec, 1)
    m = smr.Model(w, requires_grad=False)
    with torch.no_grad():
        assert tuple(m.forward(rng(12).normal(size=(1, 64, 64))).shape) == (1, 64, 64)
        # 40 x 50 pads to 64 x 64 and crops back
        assert tuple(m.forward(rng(13).normal(size=(1, 40, 50))).shape) == (1, 40, 50)


def test_model_gradients_match_finite_differences():
    """Autograd through the restated model against central differences of
    the float64 loss at 32 x 32 (the smallest size the strides allow)."""
    spec = smr.model_spec(1, 1, 0)
    w = smr.random_weights(spec, 2)
    img = rng(14).normal(0.5, 0.2, size=(1, 32, 32))
    mask = (rng(15).uniform(size=(1, 32, 32)) < 0.3).astype(np.float64)
    lo, _, grads = smr.forward_backward(w, img, mask)
    probes = [("l0_cba.conv.weight", (3, 0, 1, 2)), ("l6_lkr_1.dw.conv.weight", (5, 0, 3, 3)),
              ("l9_ctx.gate_conv.bias", (7,)), ("l15_agg.fuse.norm.weight", (4,)),
              ("l17_head.pred.bias", (2,)), ("l12_fuse.gate_dw.conv.weight", (9, 0, 0, 1)),
              ("l2_lkr.pw2.norm.bias", (11,))]

    def loss_at(name, idx, delta):
        w2 = {k: v.astype(np.float64) for k, v in w.items()}
        w2[name] = w2[name].copy()
        w2[name][idx] += delta
        m = smr.Model(w2, requires_grad=False)
        with torch.no_grad():
            z = m.forward(img).numpy()
        return smr.dice_bce_forward(z, mask).total

    for name, idx in probes:
        h = 1e-5
        fd = (loss_at(name, idx, h) - loss_at(name, idx, -h)) / (2 * h)
        g = grads[name][idx]
        assert abs(fd - g) <= 2e-5 * abs(fd) + 1e-8, (name, fd, g)


# ---- AdamW ---------------------------------------------------------------------
def test_adamw_first_step_closed_form():
    """Step 1 from zero moments: m = (1-b1) g, v = (1-b2) g^2, so the
    update is lr * g / (|g| + eps') = lr * sign(g) for |g| >> eps, after
    the decoupled decay theta *= (1 - lr*wd) (adamw.cpp:80-104)."""
    r = rng(16)
    th = r.normal(size=1000).astype(F32)
    g = (r.normal(size=1000) * 10.0 ** r.uniform(-3, 1, size=1000)).astype(F32)
    t1, m1, v1 = smr.adamw_step(th, g, np.zeros(1000, F32), np.zeros(1000, F32), 1)
    # the hyper-parameters are fp32 constants in the reference
    lr, wd, eps = float(F32(1e-3)), float(F32(1e-2)), float(F32(1e-8))
    b1, b2 = float(F32(0.9)), float(F32(0.999))
    exp = th.astype(np.float64) * (1 - lr * wd) - lr * np.sign(g)
    np.testing.assert_allclose(t1, exp, rtol=0, atol=2e-6)
    np.testing.assert_allclose(m1, (1 - b1) * g.astype(np.float64), rtol=1e-6)
    np.testing.assert_allclose(v1, (1 - b2) * g.astype(np.float64) ** 2, rtol=1e-6)
    # a later step against the float64 evaluation of the same formula
    t2, m2, v2 = smr.adamw_step(t1, g, m1, v1, 2)
    m64 = b1 * m1 + (1 - b1) * g.astype(np.float64)
    v64 = b2 * v1 + (1 - b2) * g.astype(np.float64) ** 2
    th64 = t1 * (1 - lr * wd) - (lr / (1 - b1 ** 2)) * m64 / (
        np.sqrt(v64) / math.sqrt(1 - b2 ** 2) + eps)
    np.testing.assert_allclose(t2, th64, rtol=1e-6, atol=1e-7)


def test_clip_coefficient():
    g = [np.full(3, 2.0, F32), np.full(1, 2.0, F32)]  # norm 4
    assert smr.grad_norm(g) == F32(4.0)
    assert smr.clip_coef(smr.grad_norm(g), 2.0) == F32(0.5)
    assert smr.clip_coef(F32(1.5), 2.0) is None


# ---- RLE and .soar ---------------------------------------------------------------
def test_rle_hand_checked():
    m = np.array([[1, 0, 0], [1, 1, 0], [0, 0, 1]], np.uint8)
    assert smr.encode_rle(m, 3, 3) == "1 2 5 1 9 1"
    # a run continues across a column boundary
    assert smr.encode_rle(np.array([[0, 1], [1, 1]], np.uint8), 2, 2) == "2 3"
    assert smr.encode_rle(np.zeros((4, 5), np.uint8), 4, 5) == ""
    assert smr.encode_rle(np.ones((4, 5), np.uint8), 4, 5) == "1 20"
    # non-square: H=2, W=3, column-major positions
    assert smr.encode_rle(np.array([[0, 0, 1], [0, 1, 1]], np.uint8), 2, 3) == "4 3"


def test_host_rle_encoder_matches_oracle():
    """soar_encode_rle (the host library's encoder, no device needed) against
    the column-scan restatement: random masks with nonzero values other than
    1, widths that are not multiples of the encoder's 8-column words, runs
    that cross column boundaries, empty and full masks."""
    import soar_model as sm
    try:
        sm.lib()
    except Exception as e:  # the host library is not built
        pytest.skip(f"libsoar_host.so not loadable: {e}")
    r = np.random.default_rng(11)
    for h, w in ((1, 1), (1, 9), (9, 1), (3, 3), (8, 8), (9, 17), (64, 64), (65, 63),
                 (130, 200), (5, 1000), (1000, 5), (300, 301)):
        for p in (0.0, 0.02, 0.5, 0.98, 1.0):
            on = r.uniform(size=(h, w)) < p
            m = (on * r.integers(1, 4, size=(h, w))).astype(np.uint8)
            assert sm.encode_rle(m) == smr.encode_rle(on.astype(np.uint8), h, w), (h, w, p)
    # vertical stripes: every run ends at the bottom of a column and joins
    # the next column's run
    m = np.zeros((4, 6), np.uint8)
    m[:, 1:3] = 1
    m[2:, 4] = 1
    m[:1, 5] = 1
    assert sm.encode_rle(m) == smr.encode_rle(m, 4, 6) == "5 8 19 3"


def test_soar_file_layout(tmp_path):
    p = tmp_path / "w.soar"
    named = [("a.weight", np.arange(6, dtype=F32).reshape(2, 3)), ("b", np.array([1.5], F32))]
    smr.write_soar(p, named, variant=2)
    raw = p.read_bytes()
    assert struct.unpack("<4I", raw[:16]) == (0x534F4152, 1, 2, 2)
    assert raw[16:24] == b"a.weight" and raw[24:144] == b"\0" * 120
    assert struct.unpack("<I4IQ", raw[144:172]) == (2, 2, 3, 1, 1, 24)
    assert len(raw) == 16 + (156 + 24) + (156 + 4)
    hdr, items = smr.read_soar(p)
    assert hdr == (0x534F4152, 1, 2, 2)
    assert items[0][0] == "a.weight" and items[0][2] == (2, 3, 1, 1)
    np.testing.assert_array_equal(items[0][3], named[0][1].ravel())
    np.testing.assert_array_equal(items[1][3], named[1][1])
