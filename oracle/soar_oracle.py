"""ctypes wrapper of the CPU oracle (oracle/soar_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as the computation under test.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.environ.get("SOAR_ORACLE_BUILD") or os.path.join(HERE, "build"),
                        "libsoar_oracle.so")

_F = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_D = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_I64 = ctypes.c_int64
_LIB = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def _opt(nd):
    """ndpointer that also accepts None."""
    class _Opt:
        @classmethod
        def from_param(cls, obj):
            if obj is None:
                return None
            return nd.from_param(obj)
    return _Opt


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_splitmix64_at.restype = ctypes.c_uint64
        L.orc_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_stream_key.restype = ctypes.c_uint64
        L.orc_stream_key.argtypes = [ctypes.c_uint64, ctypes.c_uint32]
        L.orc_fill_normal.argtypes = [_F, _I64, ctypes.c_uint64, ctypes.c_uint32,
                                      ctypes.c_double, ctypes.c_double]
        L.orc_fill_uniform.argtypes = [_F, _I64, ctypes.c_uint64, ctypes.c_uint32,
                                       ctypes.c_double, ctypes.c_double]
        L.orc_fill_stress.argtypes = [_F, _I64, ctypes.c_uint64] + [ctypes.c_double] * 5
        L.orc_gn_stats_f64.argtypes = [_F, _I64, _I64, _I64, _I64, _opt(_D), _opt(_D)]
        L.orc_gn_silu_fwd_f64.argtypes = [_F, _opt(_F), _opt(_F), _I64, _I64, _I64, _I64,
                                          ctypes.c_double, ctypes.c_int, ctypes.c_int,
                                          _opt(_D), _opt(_D), _opt(_D)]
        L.orc_gn_silu_bwd_f64.argtypes = [_F, _F, _opt(_F), _opt(_F), _D, _D, _I64, _I64,
                                          _I64, _I64, ctypes.c_int, ctypes.c_int, _opt(_D),
                                          _opt(_D), _opt(_D)]
        L.ref_group_norm_forward_f32.argtypes = [_F, _opt(_F), _opt(_F), _F, _F, _F, _I64,
                                                 _I64, _I64, ctypes.c_float]
        L.ref_silu_forward_f32.argtypes = [_F, _F, _I64]
        L.ref_silu_backward_f32.argtypes = [_F, _F, _F, _I64]
        L.ref_group_norm_backward_f32.argtypes = [_F, _F, _opt(_F), _F, _F, _opt(_F),
                                                  _opt(_F), _opt(_F), _I64, _I64, _I64]
        L.ref_add_f32.argtypes = [_F, _F, _F, _I64]
        L.ref_accumulate_f32.argtypes = [_F, _F, _I64]
        L.orc_conv1x1_fwd_f64.argtypes = [_F, _F, _opt(_F), _I64, _I64, _I64, _I64, _D]
        L.ref_conv1x1_fwd_f32.argtypes = [_F, _F, _opt(_F), _F, _I64, _I64, _I64]
        L.orc_conv1x1_bwd_f64.argtypes = [_F, _F, _F, _I64, _I64, _I64, _I64, _opt(_D),
                                          _opt(_D), _opt(_D)]
        L.ref_conv1x1_bwd_f32.argtypes = [_F, _F, _F, _opt(_F), _opt(_F), _opt(_F), _I64, _I64,
                                          _I64]
        _DWS = [_I64] * 9
        L.orc_dw_fwd_f64.argtypes = [_F, _F, _opt(_F), _I64] + _DWS + [_D]
        L.orc_dw_bwd_f64.argtypes = [_F, _F, _F, _I64] + _DWS + [_opt(_D), _opt(_D), _opt(_D)]
        L.ref_dw_fwd_f32.argtypes = [_F, _F, _opt(_F), _F] + _DWS
        L.ref_dw_bwd_f32.argtypes = [_F, _F, _F, _opt(_F), _opt(_F), _opt(_F)] + _DWS
        L.ref_gn_silu_fwd_bwd_f32.argtypes = [_F, _opt(_F), _opt(_F), _opt(_F), _I64, _I64,
                                              _I64, _I64, ctypes.c_float, ctypes.c_int, _F,
                                              _F, _F, _F, _F, _F, _opt(_F), _opt(_F),
                                              ctypes.POINTER(ctypes.c_double),
                                              ctypes.POINTER(ctypes.c_double)]
        _LIB = L
    return _LIB


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


# ---- synthetic inputs -------------------------------------------------------

def fill_normal(n, seed, stream, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(out, n, seed, stream, mean, std)
    return out


def fill_uniform(n, seed, stream, lo, hi):
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_uniform(out, n, seed, stream, lo, hi)
    return out


def fill_stress(n, seed, center=1e3, std=1e-2, p=1e-3, out_mean=0.0, out_std=50.0):
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_stress(out, n, seed, center, std, p, out_mean, out_std)
    return out


# ---- float64 truth ------------------------------------------------------------

def gn_stats_f64(x, N, C, HW, G):
    mean = np.empty(N * G)
    var = np.empty(N * G)
    rc = lib().orc_gn_stats_f64(_f32(x).reshape(-1), N, C, HW, G, mean, var)
    assert rc == 0, rc
    return mean, var


def gn_silu_fwd_f64(x, gamma, beta, N, C, HW, G, eps, silu=True, residual=False,
                    want_y=True):
    x = _f32(x).reshape(-1)
    y = np.empty(N * C * HW) if want_y else None
    mean = np.empty(N * G)
    rstd = np.empty(N * G)
    rc = lib().orc_gn_silu_fwd_f64(x, _f32(gamma), _f32(beta), N, C, HW, G, float(eps),
                                   int(silu), int(residual), y, mean, rstd)
    assert rc == 0, rc
    return y, mean, rstd


def gn_silu_bwd_f64(dy, x, gamma, beta, mean, rstd, N, C, HW, G, silu=True,
                    residual=False, want_dx=True):
    dx = np.empty(N * C * HW) if want_dx else None
    dgamma = np.empty(C)
    dbeta = np.empty(C)
    rc = lib().orc_gn_silu_bwd_f64(_f32(dy).reshape(-1), _f32(x).reshape(-1), _f32(gamma),
                                   _f32(beta), np.ascontiguousarray(mean, dtype=np.float64),
                                   np.ascontiguousarray(rstd, dtype=np.float64), N, C, HW, G,
                                   int(silu), int(residual), dx, dgamma, dbeta)
    assert rc == 0, rc
    return dx, dgamma, dbeta


# ---- fp32 statement of the reference CPU path -----------------------------------

def ref_gn_forward_f32(x, gamma, beta, C, HW, G, eps):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    means = np.empty(G, dtype=np.float32)
    rstds = np.empty(G, dtype=np.float32)
    rc = lib().ref_group_norm_forward_f32(x, _f32(gamma), _f32(beta), y, means, rstds, C,
                                          HW, G, eps)
    assert rc == 0, rc
    return y, means, rstds


def ref_silu_forward_f32(x):
    x = _f32(x).reshape(-1)
    y = np.empty_like(x)
    lib().ref_silu_forward_f32(x, y, x.size)
    return y


def ref_silu_backward_f32(gy, x):
    x = _f32(x).reshape(-1)
    gx = np.empty_like(x)
    lib().ref_silu_backward_f32(_f32(gy).reshape(-1), x, gx, x.size)
    return gx


def ref_gn_backward_f32(go, x, gamma, means, rstds, C, HW, G):
    x = _f32(x).reshape(-1)
    gx = np.empty_like(x)
    gw = np.empty(C, dtype=np.float32)
    gb = np.empty(C, dtype=np.float32)
    rc = lib().ref_group_norm_backward_f32(_f32(go).reshape(-1), x, _f32(gamma), _f32(means),
                                           _f32(rstds), gx, gw, gb, C, HW, G)
    assert rc == 0, rc
    return gx, gw, gb


def ref_gn_silu_fwd_bwd_f32(x, gamma, beta, dy, N, C, HW, G, eps, residual=False):
    """The reference's unfused per-sample GN -> SiLU [-> add] forward and
    backward; returns a dict of outputs plus fwd/bwd wall seconds."""
    x = _f32(x).reshape(-1)
    n = x.size
    out = {k: np.empty(n, dtype=np.float32) for k in ("gn_out", "y", "dz", "dx")}
    out["mean"] = np.empty(N * G, dtype=np.float32)
    out["rstd"] = np.empty(N * G, dtype=np.float32)
    out["dgamma"] = np.empty(C, dtype=np.float32)
    out["dbeta"] = np.empty(C, dtype=np.float32)
    tf, tb = ctypes.c_double(), ctypes.c_double()
    rc = lib().ref_gn_silu_fwd_bwd_f32(x, _f32(gamma), _f32(beta),
                                       None if dy is None else _f32(dy).reshape(-1), N, C, HW,
                                       G, eps, int(residual), out["gn_out"], out["y"],
                                       out["mean"], out["rstd"], out["dz"], out["dx"],
                                       out["dgamma"], out["dbeta"], ctypes.byref(tf),
                                       ctypes.byref(tb))
    assert rc == 0, rc
    out["fwd_s"] = tf.value
    out["bwd_s"] = tb.value
    return out


# ---- pointwise convolution ------------------------------------------------------

def conv1x1_fwd_f64(x, w, b, N, C_in, C_out, HW):
    y = np.empty(N * C_out * HW)
    rc = lib().orc_conv1x1_fwd_f64(_f32(x).reshape(-1), _f32(w).reshape(-1), _f32(b), N, C_in,
                                   C_out, HW, y)
    assert rc == 0, rc
    return y


def ref_conv1x1_fwd_f32(x, w, b, C_in, C_out, HW):
    y = np.empty(C_out * HW, dtype=np.float32)
    lib().ref_conv1x1_fwd_f32(_f32(x).reshape(-1), _f32(w).reshape(-1), _f32(b), y, C_in, C_out,
                              HW)
    return y


def conv1x1_bwd_f64(dz, x, w, N, C_in, C_out, HW, want=("dx", "dw", "db")):
    dx = np.empty(N * C_in * HW) if "dx" in want else None
    dw = np.empty(C_out * C_in) if "dw" in want else None
    db = np.empty(C_out) if "db" in want else None
    rc = lib().orc_conv1x1_bwd_f64(_f32(dz).reshape(-1), _f32(x).reshape(-1),
                                   _f32(w).reshape(-1), N, C_in, C_out, HW, dx, dw, db)
    assert rc == 0, rc
    return dx, dw, db


def ref_conv1x1_bwd_f32(go, x, w, C_in, C_out, HW, grad_in=None, grad_weight=None,
                        grad_bias=None):
    """Accumulates into the given arrays (zeros when None)."""
    gi = np.zeros(C_in * HW, np.float32) if grad_in is None else grad_in
    gw = np.zeros(C_out * C_in, np.float32) if grad_weight is None else grad_weight
    gb = np.zeros(C_out, np.float32) if grad_bias is None else grad_bias
    lib().ref_conv1x1_bwd_f32(_f32(go).reshape(-1), _f32(x).reshape(-1), _f32(w).reshape(-1),
                              gi, gw, gb, C_in, C_out, HW)
    return gi, gw, gb


# ---- depthwise convolution --------------------------------------------------------

def dw_out_size(H, K, pad, stride, dil):
    """Conv2d::forward's output size (src/nn/layers.cpp:330-332)."""
    return (H + 2 * pad - (dil * (K - 1) + 1)) // stride + 1


def dw_fwd_f64(x, w, b, N, C, H, W, K, pad, stride, dil):
    Ho, Wo = dw_out_size(H, K, pad, stride, dil), dw_out_size(W, K, pad, stride, dil)
    y = np.empty(N * C * Ho * Wo)
    rc = lib().orc_dw_fwd_f64(_f32(x).reshape(-1), _f32(w).reshape(-1), _f32(b), N, C, H, W,
                              Ho, Wo, K, pad, stride, dil, y)
    assert rc == 0, rc
    return y.reshape(N, C, Ho, Wo)


def dw_bwd_f64(dy, x, w, N, C, H, W, K, pad, stride, dil):
    Ho, Wo = dw_out_size(H, K, pad, stride, dil), dw_out_size(W, K, pad, stride, dil)
    dx = np.empty(N * C * H * W)
    dw = np.empty(C * K * K)
    db = np.empty(C)
    rc = lib().orc_dw_bwd_f64(_f32(dy).reshape(-1), _f32(x).reshape(-1), _f32(w).reshape(-1),
                              N, C, H, W, Ho, Wo, K, pad, stride, dil, dx, dw, db)
    assert rc == 0, rc
    return dx.reshape(N, C, H, W), dw.reshape(C, K, K), db


def ref_dw_fwd_f32(x, w, b, C, H, W, K, pad, stride, dil):
    Ho, Wo = dw_out_size(H, K, pad, stride, dil), dw_out_size(W, K, pad, stride, dil)
    y = np.empty(C * Ho * Wo, np.float32)
    lib().ref_dw_fwd_f32(_f32(x).reshape(-1), _f32(w).reshape(-1), _f32(b), y, C, H, W, Ho, Wo,
                         K, pad, stride, dil)
    return y.reshape(C, Ho, Wo)


def ref_dw_bwd_f32(dy, x, w, C, H, W, K, pad, stride, dil, grad_in=None):
    Ho, Wo = dw_out_size(H, K, pad, stride, dil), dw_out_size(W, K, pad, stride, dil)
    gi = np.zeros(C * H * W, np.float32) if grad_in is None else grad_in
    gw = np.zeros(C * K * K, np.float32)
    gb = np.zeros(C, np.float32)
    lib().ref_dw_bwd_f32(_f32(dy).reshape(-1), _f32(x).reshape(-1), _f32(w).reshape(-1), gi, gw,
                         gb, C, H, W, Ho, Wo, K, pad, stride, dil)
    return gi.reshape(C, H, W), gw.reshape(C, K, K), gb
