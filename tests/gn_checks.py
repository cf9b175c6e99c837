"""Checks of GroupNorm results at full size that the value bars cannot
make (shared by the GPU parity tests and the CPU test that plants mistakes
in oracle-made gradients to show the checks catch them)."""
import numpy as np

# The GroupNorm correction of dx at full size.  dx = r (gamma dz - (S1 +
# xhat S2) / M) [+ dy] (src/nn/layers.cpp:606-616): at 2^24-element units
# r S1 / M and r S2 / M are ~1e-7..1e-6, hundreds of times under the 1e-4
# value bar, so the value checks cannot see a dropped or wrong S1 / S2
# term.  These checks take the main term out first.
#   DX_ULPS: fp32 rounding budget, in units of 2^-24, of the device's main
#   term r gamma dz (the sigmoid from v_exp_f32 / v_rcp_f32, the dz product,
#   the rounding of xhat propagated through the SiLU derivative, the final
#   fma); CORR_REL: the device's S1, S2 are sums of its fp32 dz, so each of
#   the two correction terms may differ by that much relative from the exact
#   ones (the slack scales with |S1| + |xhat S2|, not with their sum, which
#   cancels near xhat = -S1 / S2).  A wrong S2 term changes c by r |xhat S2| / M, about 20x this
#   budget at |xhat| = 1 at config 3, and the fit below is exact to ~1e-4
#   relative, so a dropped, sign-flipped or half-scaled term fails both.
DX_ULPS = 32
CORR_REL = 1e-3       # relative slack on each correction term (the device sums fp32 dz)
FIT_REL = 1e-2        # fitted a, b against -r S1 / M, -r S2 / M
INVARIANT_REL = 1e-6  # sum(xhat dx) against r S2 (1 - sum(xhat^2) / M), over sum|xhat dx|


def check_dx_correction(dx, x, dy, gamma, beta, mean, rstd, G, what, silu=True,
                        residual=False):
    """Per unit (n, g), in float64 on the device with the statistics the
    kernels used (mean: the effective mean, float64 [N*G]; rstd [N*G]):
      c = dx - r gamma dz [- dy] against -r (S1 + xhat S2) / M elementwise,
          within DX_ULPS * 2^-24 of the main term's scale + CORR_REL r (|S1| +
          |xhat S2|) / M;
      the least-squares fit c ~ a + b xhat: a against -r S1 / M and b
          against -r S2 / M within FIT_REL;
      sum(xhat dx_gn) = r S2 (1 - sum(xhat^2) / M) (= r S2 eps / (var + eps)
          in exact arithmetic) within INVARIANT_REL * sum|xhat dx_gn|.
    Returns the largest elementwise error over its bound (for reports)."""
    import torch
    dev_ = x.device
    N, C = x.shape[0], x.shape[1]
    x3, dy3, dx3 = x.view(N, C, -1), dy.view(N, C, -1), dx.view(N, C, -1)
    HW = x3.shape[2]
    cpg = C // G
    M = float(cpg * HW)
    u32 = 2.0 ** -24
    mean = torch.as_tensor(np.asarray(mean, np.float64), device=dev_)
    rstd = torch.as_tensor(np.asarray(rstd, np.float64), device=dev_)
    g64 = gamma.double() if gamma is not None else torch.ones(C, dtype=torch.float64,
                                                              device=dev_)
    b64 = beta.double() if beta is not None else torch.zeros(C, dtype=torch.float64,
                                                             device=dev_)
    worst = 0.0
    for n in range(N):
        for g in range(G):
            u = n * G + g
            cs = slice(g * cpg, (g + 1) * cpg)
            r = rstd[u]
            xh = (x3[n, cs].double() - mean[u]) * r
            gm, bt = g64[cs, None], b64[cs, None]
            dyu = dy3[n, cs].double()
            z = gm * xh + bt
            if silu:
                s = torch.sigmoid(z)
                dz = dyu * s * (1 + z * (1 - s))
            else:
                dz = dyu
            gdz = gm * dz
            S1, S2 = gdz.sum(), (gdz * xh).sum()
            dxu = dx3[n, cs].double()
            dxg = dxu - (dyu if residual else 0.0)
            c = dxg - r * gdz
            ct = -r * (S1 + xh * S2) / M
            scale = r * gm.abs() * dyu.abs() * (1 + z.abs() + gm.abs() * xh.abs())
            terms = r * (S1.abs() + (xh * S2).abs()) / M  # |c|'s two terms, before they cancel
            # (with the residual, dx's last rounding is that of dx_gn + dy)
            rnd = dxg.abs() + (dxu.abs() if residual else 0.0)
            bound = DX_ULPS * u32 * (scale + rnd) + CORR_REL * terms + 1e-30
            q = (c - ct).abs() / bound
            ratio = float(q.max())
            worst = max(worst, ratio)
            if ratio > 1.0:
                i = int(q.argmax())
                pick = lambda t: float(t.reshape(-1)[i])
                raise AssertionError(
                    f"{what} unit {u}: correction error {ratio:.3g} x its bound at {i}: c "
                    f"{pick(c):.6e} vs {pick(ct):.6e}, main {pick(r * gdz):.3e}, dx "
                    f"{pick(dxg):.6e}, xhat {pick(xh):.4f}, z {pick(z):.4f}, dy {pick(dyu):.3e}")
            # least-squares fit c ~ a + b xhat
            xm, cm = xh.mean(), c.mean()
            b = float(((xh - xm) * (c - cm)).sum() / ((xh - xm) ** 2).sum())
            a = float(cm - b * xm)
            at, bt_ = float(-r * S1 / M), float(-r * S2 / M)
            assert abs(a - at) <= FIT_REL * abs(at) + 1e-15, f"{what} unit {u}: a {a} vs {at}"
            assert abs(b - bt_) <= FIT_REL * abs(bt_) + 1e-15, f"{what} unit {u}: b {b} vs {bt_}"
            # sum(xhat dx_gn) = r S2 (1 - sum xhat^2 / M)
            p = xh * dxg
            want = float(r * S2 * (1 - (xh * xh).sum() / M))
            got = float(p.sum())
            tol = INVARIANT_REL * float(p.abs().sum())
            assert abs(got - want) <= tol, f"{what} unit {u}: sum(xhat dx) {got} vs {want} +- {tol}"
    return worst
