"""CPU restatement of the SOAR model's training step and prediction.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP
model path (libsoar_host.so), never as the computation under test.

What it restates (reference: pomagrenate/soar.cpp):
  * SOARModel construction and forward, every block and layer
    (src/nn/soar_model.cpp:175-417, src/nn/blocks.cpp:429-620,
    src/nn/layers.cpp:294-1345), in float64 on the CPU with torch's
    functional operators; parameter names and order as named_parameters()
    lists them (include/soar/nn/module.hpp:59-70, std::map order).
  * DiceBCELoss forward (losses.cpp:80-122,207-262,464-478 with the
    device-path values of loss_kernels.cu:51-69,141-174) and its backward
    formula (loss_kernels.cu:212-252), which is applied as given (it omits
    the forward's 1e-7 in the Dice denominator), then back-propagated
    through the model with torch autograd.
  * AdamW::clip_grad_norm and AdamW::step (adamw.cpp:28-108) as scalar
    float32 IEEE arithmetic (numpy float32, no fused multiply-add).
  * Predictor::predict and encode_rle (predictor.cpp:10-85).
  * The .soar weight file (soar_model.cpp:427-523).

How each part is pinned (tests/test_oracle_model.py): the bilinear resize,
pixel shuffle, pad and the loss against brute-force loops of the
reference's own formulas; the model's gradients against central finite
differences of the float64 loss; torch's conv2d / group_norm against the
oracle's C statements (oracle/soar_oracle.c) through the CBA blocks; AdamW
against a closed form (first step moves every weight by lr * sign(g) after
decay); RLE against hand-checked strings; the .soar reader/writer by a
round trip and the byte layout.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

F32 = np.float32
GN_EPS = float(F32(1e-5))  # GroupNorm eps, an fp32 constant in the reference


def select_group_count(c: int, max_groups: int = 8) -> int:
    """Largest divisor of c not above max_groups (layers.hpp:9-14)."""
    for g in range(min(max_groups, c), 0, -1):
        if c % g == 0:
            return g
    return 1


def autopad(k: int, p: int = -1, d: int = 1) -> int:
    """Conv2d padding when p < 0 (layers.hpp:16-19)."""
    if d > 1:
        k = d * (k - 1) + 1
    return k // 2 if p < 0 else p


# ---------------------------------------------------------------------------
# Architecture: parameter specs in named_parameters() order
# ---------------------------------------------------------------------------
ARCH = {  # soar_model.cpp:182-208
    0: (16, 32, 32, 64, 64, 128, 128, 256, 256, 256, 128, 128, 64, 64, 32, 32, 16, 16, 1, 1, 2, 1, 1, 1),
    1: (24, 48, 48, 96, 96, 192, 192, 384, 384, 384, 192, 192, 96, 96, 48, 48, 24, 24, 1, 2, 3, 2, 1, 1),
    2: (32, 64, 64, 128, 128, 256, 256, 512, 512, 512, 256, 256, 128, 128, 64, 64, 32, 32, 2, 3, 5, 3, 1, 1),
    3: (32, 64, 64, 160, 160, 320, 320, 640, 640, 640, 320, 320, 160, 160, 64, 64, 32, 32, 2, 3, 7, 4, 2, 1),
    4: (40, 80, 80, 192, 192, 384, 384, 768, 768, 768, 384, 384, 192, 192, 80, 80, 40, 40, 2, 4, 8, 5, 2, 2),
}


class _Spec:
    """A module tree that records parameters like Module does: own
    parameters sorted by name, then submodules sorted by name."""

    def __init__(self):
        self.params = {}   # name -> shape
        self.subs = {}     # name -> _Spec
        self.init = {}     # name -> "zeros" / "ones" / ("fill", v) (reference init)

    def sub(self, name):
        s = _Spec()
        self.subs[name] = s
        return s

    def named(self, prefix=""):
        out = []
        for n in sorted(self.params):
            out.append((f"{prefix}.{n}" if prefix else n, self.params[n], self.init.get(n)))
        for n in sorted(self.subs):
            out.extend(self.subs[n].named(f"{prefix}.{n}" if prefix else n))
        return out


def _conv_spec(s, c1, c2, k, g=1, bias=True):
    s.params["weight"] = (c2, c1 // g, k, k)
    s.init["weight"] = "kaiming"
    if bias:
        s.params["bias"] = (c2,)
        s.init["bias"] = "zeros"


def _cba_spec(s, c1, c2, k=1, g=1):
    _conv_spec(s.sub("conv"), c1, c2, k, g, bias=False)
    n = s.sub("norm")
    n.params["weight"] = (c2,)
    n.params["bias"] = (c2,)
    n.init["weight"] = "ones"
    n.init["bias"] = "zeros"
    return s


def _lkr_h(c, e=2.0):
    return max(int(F32(c) * F32(e)), 8)


def model_spec(in_channels=1, num_classes=1, variant=0):
    """[(name, shape, init)] of SOARModel in named_parameters() order."""
    a = ARCH[variant]
    c0, c1, c2, c3, c4, c5, c6, c7, c8, c9, c10, c11, c12, c13, c14, c15, c16, c17 = a[:18]
    n2, n4, n6, n8, n11, n13 = a[18:]
    m = _Spec()
    _cba_spec(m.sub("l0_cba"), in_channels, c0, 3)

    def down(name, ci, co):
        d = m.sub(name)
        _cba_spec(d.sub("dw"), ci, ci, 3, ci)
        _cba_spec(d.sub("pw"), ci, co, 1)

    def lkr(spec, c, k):
        h = _lkr_h(c)
        _cba_spec(spec.sub("dw"), c, c, k, c)
        _cba_spec(spec.sub("pw1"), c, h, 1)
        p2 = _cba_spec(spec.sub("pw2"), h, c, 1)
        p2.subs["norm"].init["weight"] = "zeros"  # blocks.cpp:469-470

    def stack(base, n, c, k, always=False):
        for i in range(n):
            lkr(m.sub(base if (n == 1 and not always) else f"{base}_{i}"), c, k)

    def fuse(name, cl, cs, co):
        f = m.sub(name)
        _cba_spec(f.sub("low"), cl, co)
        _cba_spec(f.sub("skip"), cs, co)
        _cba_spec(f.sub("gate_dw"), co, co, 3, co)
        _conv_spec(f.sub("gate_conv"), co, co, 1)
        _cba_spec(f.sub("out_dw"), co, co, 3, co)
        _cba_spec(f.sub("out_pw"), co, co)

    down("l1_down", c0, c1)
    stack("l2_lkr", n2, c2, 5)
    down("l3_down", c2, c3)
    stack("l4_lkr", n4, c4, 7)
    down("l5_down", c4, c5)
    stack("l6_lkr", n6, c6, 7, always=True)
    down("l7_down", c6, c7)
    stack("l8_lkr", n8, c8, 7)
    ctx = m.sub("l9_ctx")
    h = c9 // 2
    _cba_spec(ctx.sub("cv1"), c8, h)
    for i in range(3):
        _cba_spec(ctx.sub(f"branch_{i}"), h, h, 3, h)
    _cba_spec(ctx.sub("cv2"), h * 4, c9)
    _conv_spec(ctx.sub("gate_conv"), c8, c9, 1)
    fuse("l10_fuse", c9, c6, c10)
    stack("l11_lkr", n11, c11, 7)
    fuse("l12_fuse", c11, c4, c12)
    stack("l13_lkr", n13, c13, 7)
    fuse("l14_fuse", c13, c2, c14)
    agg = m.sub("l15_agg")
    p = max(c15 // 2, 8)
    for i, ch in enumerate((c14, c13, c11)):
        _cba_spec(agg.sub(f"proj_{i}"), ch, p)
    _cba_spec(agg.sub("fuse"), p * 3, c15)
    fuse("l16_fuse", c15, c0, c16)
    head = m.sub("l17_head")
    _cba_spec(head.sub("refine_dw"), c16, c16, 3, c16)
    _cba_spec(head.sub("refine_pw"), c16, c17)
    _conv_spec(head.sub("pred"), c17, num_classes * 4, 1)
    head.subs["pred"].init["bias"] = ("fill", float(-F32(math.log(F32(1.0 - F32(0.01)) / F32(0.01)))))
    return m.named()


def random_weights(spec, seed):
    """Random float32 weights for a spec (not the reference's initial
    values: every path, including LKR's zero-initialised pw2 scale, gets a
    non-trivial value)."""
    r = np.random.default_rng(seed)
    w = {}
    for name, shape, _ in spec:
        if name.endswith("norm.weight"):
            v = r.uniform(0.5, 1.5, size=shape)
        elif name.endswith("norm.bias"):
            v = r.normal(0.0, 0.1, size=shape)
        elif name.endswith("bias"):
            v = r.normal(0.0, 0.1, size=shape)
        else:
            fan_in = int(np.prod(shape[1:]))
            b = 1.0 / math.sqrt(fan_in)
            v = r.uniform(-b, b, size=shape)
        w[name] = v.astype(F32)
    return w


# ---------------------------------------------------------------------------
# Forward (float64)
# ---------------------------------------------------------------------------
def resize_bilinear(x, th, tw):
    """Upsample to round(H*scale) with scale = th/H (blocks.cpp:420-427,
    layers.cpp:1073-1150): half-pixel, no corner alignment, source index
    clamped at 0; torch's bilinear with align_corners=False is the same map
    (pinned against the reference's loop)."""
    H, W = x.shape[-2:]
    if H == th and W == tw:
        return x
    scale = F32(th) / F32(H)
    ho = int(round(float(F32(H) * scale)))
    wo = int(round(float(F32(W) * scale)))
    return F.interpolate(x, size=(ho, wo), mode="bilinear", align_corners=False)


def pad_spatial(x, ph, pw):
    """Reflect (ph < H and pw < W) or edge-repeat padding of [1,C,H,W]."""
    H, W = x.shape[-2:]
    reflect = ph < H and pw < W

    def src(n, p):
        idx = np.arange(n + p)
        over = idx >= n
        idx[over] = (2 * (n - 1) - idx[over]) if reflect else n - 1
        return torch.as_tensor(idx)

    return x[:, :, src(H, ph)][:, :, :, src(W, pw)]


class Model:
    """Forward of SOARModel over a dict of float64 leaf tensors."""

    def __init__(self, weights, in_channels=1, num_classes=1, variant=0, requires_grad=True):
        self.a = ARCH[variant]
        self.nc = num_classes
        self.P = {k: torch.tensor(np.asarray(v, dtype=np.float64), requires_grad=requires_grad)
                  for k, v in weights.items()}

    def conv(self, pre, x, k=1, s=1, p=-1, d=1, g=1):
        w = self.P[pre + ".weight"]
        b = self.P.get(pre + ".bias")
        return F.conv2d(x, w, b, stride=s, padding=autopad(k, p, d), dilation=d, groups=g)

    def cba(self, pre, x, k=1, s=1, d=1, g=1, act=True):
        """Conv2d (no bias) -> GroupNorm -> SiLU (blocks.cpp:429-445)."""
        z = self.conv(pre + ".conv", x, k, s, -1, d, g)
        c2 = z.shape[1]
        y = F.group_norm(z, select_group_count(c2), self.P[pre + ".norm.weight"],
                         self.P[pre + ".norm.bias"], eps=GN_EPS)
        return F.silu(y) if act else y

    def down(self, pre, x):
        c = x.shape[1]
        return self.cba(pre + ".pw", self.cba(pre + ".dw", x, 3, 2, 1, c, False))

    def lkr(self, pre, x, k):
        c = x.shape[1]
        y = self.cba(pre + ".dw", x, k, 1, 1, c, False)
        return x + self.cba(pre + ".pw2", self.cba(pre + ".pw1", y), act=False)

    def stack(self, base, n, x, k, always=False):
        for i in range(n):
            x = self.lkr(base if (n == 1 and not always) else f"{base}_{i}", x, k)
        return x

    def ctx(self, pre, x):
        """blocks.cpp:486-519."""
        y = self.cba(pre + ".cv1", x)
        h = y.shape[1]
        cat = [y] + [self.cba(f"{pre}.branch_{i}", y, 3, 1, d, h, False)
                     for i, d in enumerate((1, 3, 5))]
        out = self.cba(pre + ".cv2", torch.cat(cat, dim=1))
        pooled = x.mean(dim=(2, 3), keepdim=True)
        gate = torch.sigmoid(self.conv(pre + ".gate_conv", pooled, 1, 1, 0))
        gated = out * gate
        return x + gated if x.shape[1] == out.shape[1] else gated

    def fuse(self, pre, low, skip):
        """blocks.cpp:524-559."""
        a = self.cba(pre + ".skip", skip, act=False)
        b = resize_bilinear(self.cba(pre + ".low", low, act=False), a.shape[2], a.shape[3])
        c = a.shape[1]
        gate = torch.sigmoid(self.conv(pre + ".gate_conv",
                                       self.cba(pre + ".gate_dw", a + b, 3, 1, 1, c, False), 1, 1, 0))
        fused = gate * a + (1.0 - gate) * b
        return self.cba(pre + ".out_pw", self.cba(pre + ".out_dw", fused, 3, 1, 1, c, False))

    def agg(self, pre, inputs):
        """blocks.cpp:564-591."""
        th, tw = inputs[0].shape[2:]
        ys = []
        for i, t in enumerate(inputs):
            y = self.cba(f"{pre}.proj_{i}", t)
            if y.shape[2] != th or y.shape[3] != tw:
                y = resize_bilinear(y, th, tw)
            ys.append(y)
        return self.cba(pre + ".fuse", torch.cat(ys, dim=1))

    def head(self, pre, x):
        """blocks.cpp:596-620 (PixelShuffle r = 2, layers.cpp:928-989)."""
        c = x.shape[1]
        y = self.cba(pre + ".refine_pw", self.cba(pre + ".refine_dw", x, 3, 1, 1, c, False))
        return F.pixel_shuffle(self.conv(pre + ".pred", y, 1, 1, 0), 2)

    def forward(self, img):
        """img [C,H,W] (numpy or tensor) -> logits [nc,H,W] (soar_model.cpp:316-417)."""
        x = torch.as_tensor(np.asarray(img, dtype=np.float64))[None]
        H, W = x.shape[2:]
        ph, pw = (32 - H % 32) % 32, (32 - W % 32) % 32
        if ph or pw:
            x = pad_spatial(x, ph, pw)
        n2, n4, n6, n8, n11, n13 = self.a[18:]
        s2 = self.cba("l0_cba", x, 3, 2)
        p2 = self.stack("l2_lkr", n2, self.down("l1_down", s2), 5)
        p3 = self.stack("l4_lkr", n4, self.down("l3_down", p2), 7)
        p4 = self.stack("l6_lkr", n6, self.down("l5_down", p3), 7, always=True)
        p5 = self.stack("l8_lkr", n8, self.down("l7_down", p4), 7)
        p5c = self.ctx("l9_ctx", p5)
        d16 = self.stack("l11_lkr", n11, self.fuse("l10_fuse", p5c, p4), 7)
        d8 = self.stack("l13_lkr", n13, self.fuse("l12_fuse", d16, p3), 7)
        d4 = self.fuse("l14_fuse", d8, p2)
        agg = self.agg("l15_agg", [d4, d8, d16])
        d2 = self.fuse("l16_fuse", agg, s2)
        out = self.head("l17_head", d2)
        return out[0, :, :H, :W]


# ---------------------------------------------------------------------------
# Loss (float64 values of the reference's formulas)
# ---------------------------------------------------------------------------
@dataclass
class LossOut:
    total: float
    bce: float
    dice: float
    inter: float
    sum_p: float
    sum_y: float


def dice_bce_forward(z, y, weight=1.0, bce_weight=0.5, dice_weight=0.5, pos_weight=3.0,
                     smooth=1.0):
    """DiceBCELoss::forward with CompositeLoss(0.5, 0.5) defaults
    (losses.cpp:464-478, loss_kernels.cu:29-69,111-174)."""
    z = np.asarray(z, dtype=np.float64).ravel()
    y = np.asarray(y, dtype=np.float64).ravel()
    w = 1.0 + (pos_weight - 1.0) * y
    term = np.maximum(-z, 0.0) + np.log1p(np.exp(-np.abs(z)))
    bce = float(np.mean((1.0 - y) * z + w * term))
    p = 1.0 / (1.0 + np.exp(-z))
    inter, sp, sy = float(np.sum(p * y)), float(np.sum(p)), float(np.sum(y))
    dice = 1.0 - (2.0 * inter + smooth) / (sp + sy + smooth + 1e-7)
    total = weight * (bce_weight * bce + dice_weight * dice)
    return LossOut(total, bce, dice, inter, sp, sy)


def dice_bce_grad(z, y, lo: LossOut, go=1.0, w=1.0, bw=0.5, dw=0.5, pos_weight=3.0, smooth=1.0):
    """The backward formula of loss_kernels.cu:212-252 (float64)."""
    z = np.asarray(z, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    n = z.size
    sig = 1.0 / (1.0 + np.exp(-z))
    g = (sig * (1.0 + (pos_weight - 1.0) * y) - pos_weight * y) * (go * w * bw / n)
    denom = lo.sum_p + lo.sum_y + smooth
    numer = 2.0 * lo.inter + smooth
    d_dice_dp = (2.0 * y * denom - numer) / (denom * denom)
    g = g + (go * w * dw) * (-d_dice_dp * sig * (1.0 - sig))
    return g


def forward_backward(weights, img, mask, variant=0):
    """Loss, logits and float64 parameter gradients of one image
    (Trainer::train_step up to the optimizer, trainer.cpp:147-156)."""
    m = Model(weights, in_channels=np.asarray(img).shape[0], variant=variant)
    logits = m.forward(img)
    z = logits.detach().numpy()
    lo = dice_bce_forward(z, mask)
    gz = dice_bce_grad(z, np.asarray(mask, dtype=np.float64).reshape(z.shape), lo)
    logits.backward(torch.as_tensor(gz))
    grads = {k: v.grad.numpy().copy() for k, v in m.P.items()}
    return lo, z, grads


# ---------------------------------------------------------------------------
# AdamW (float32 scalar arithmetic, adamw.cpp:28-108)
# ---------------------------------------------------------------------------
def clip_coef(grad_norm, max_norm=2.0):
    """Scale of clip_grad_norm for a norm already rounded to float32."""
    gn = F32(grad_norm)
    if gn > F32(max_norm) and gn > F32(1e-6):
        return F32(F32(max_norm) / gn)
    return None


def grad_norm(grads):
    """sqrt of the fp64 sum of squares, rounded to float32."""
    s = 0.0
    for g in grads:
        g = np.asarray(g, dtype=np.float64).ravel()
        s += float(np.dot(g, g))
    return F32(math.sqrt(s))


def adamw_step(theta, g, m, v, step, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, wd=1e-2):
    """One AdamW update in float32, each operation rounded separately;
    returns new (theta, m, v)."""
    with np.errstate(over="ignore"):
        lr, b1, b2, eps, wd = F32(lr), F32(beta1), F32(beta2), F32(eps), F32(wd)
        bc1 = F32(1) - np.power(b1, F32(step), dtype=F32)
        bc2 = F32(1) - np.power(b2, F32(step), dtype=F32)
        sqrt_bc2 = np.sqrt(bc2, dtype=F32)
        step_size = F32(lr / bc1)
        th = np.asarray(theta, dtype=F32).copy()
        g = np.asarray(g, dtype=F32)
        if wd != 0:
            th = (th - F32(lr * wd) * th).astype(F32)
        m = (b1 * np.asarray(m, dtype=F32) + (F32(1) - b1) * g).astype(F32)
        v = (b2 * np.asarray(v, dtype=F32) + ((F32(1) - b2) * g) * g).astype(F32)
        denom = (np.sqrt(v, dtype=F32) / sqrt_bc2 + eps).astype(F32)
        th = (th - step_size * (m / denom)).astype(F32)
    return th, m, v


# ---------------------------------------------------------------------------
# Predictor
# ---------------------------------------------------------------------------
def encode_rle(mask, height, width):
    """Column-major, 1-indexed start/length runs (predictor.cpp:10-48)."""
    m = np.asarray(mask).reshape(height, width)
    col = m.T.ravel() > 0  # column-major order
    runs, i, n = [], 0, col.size
    while i < n:
        if col[i]:
            j = i
            while j < n and col[j]:
                j += 1
            runs.append(f"{i + 1} {j - i}")
            i = j
        else:
            i += 1
    return " ".join(runs)


# ---------------------------------------------------------------------------
# .soar files (soar_model.cpp:427-523)
# ---------------------------------------------------------------------------
SOAR_MAGIC = 0x534F4152


def write_soar(path, named, variant=0):
    """named: [(name, float32 array)] in file order."""
    with open(path, "wb") as f:
        f.write(struct.pack("<4I", SOAR_MAGIC, 1, variant, len(named)))
        for name, arr in named:
            a = np.ascontiguousarray(arr, dtype=F32)
            nb = name.encode()[:127]
            f.write(nb + b"\0" * (128 - len(nb)))
            shape = list(a.shape)[:4] + [1] * (4 - min(4, a.ndim))
            f.write(struct.pack("<I4IQ", a.ndim, *shape, a.nbytes))
            f.write(a.tobytes())


def read_soar(path):
    """-> (header (magic, version, variant, count), [(name, ndim, shape4, float32 array)])."""
    out = []
    with open(path, "rb") as f:
        hdr = struct.unpack("<4I", f.read(16))
        for _ in range(hdr[3]):
            name = f.read(128).split(b"\0", 1)[0].decode()
            ndim, s0, s1, s2, s3, nbytes = struct.unpack("<I4IQ", f.read(28))
            data = np.frombuffer(f.read(nbytes), dtype=F32).copy()
            out.append((name, ndim, (s0, s1, s2, s3), data))
    return hdr, out
