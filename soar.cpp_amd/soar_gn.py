"""ctypes binding of libsoar_gn.so, the MI355X GroupNorm+SiLU library.

The reference ships the same kind of thin ctypes layer over its C-ABI
(pomagrenate/soar.cpp ``soar/__init__.py:16-96``).  This one binds the
operator-level C-ABI of ``include/soar_gn.h`` and adds helpers that take
torch tensors (torch is only the device-memory and stream plumbing here:
every computation runs in the HIP kernels of ``csrc/``).

Importing this module never falls back to anything: if the library is not
built, :func:`lib` raises :class:`SoarUnavailable`.
"""
from __future__ import annotations

import ctypes
import json
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
# SOAR_LIB_DIR selects another build of the two libraries (the sanitizer
# build of `make sanitize`, for instance); the default is the in-tree lib/.
LIB_DIR = os.environ.get("SOAR_LIB_DIR") or os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libsoar_gn.so")
SYNTH_PATH = os.path.join(LIB_DIR, "libsoar_synth.so")
HEADER_PATH = os.path.join(ROOT, "include", "soar_gn.h")

SOAR_OK = 0
SOAR_EINVAL = -1
SOAR_ENOMEM = -2
SOAR_EHIP = -3
SOAR_ENODEV = -4

GN_SILU = 1
GN_RESIDUAL = 2
GN_ACCUMULATE_DX = 4
DEFER_WEIGHT_FINISH = 8
ADAMW_ZERO_GRAD = 1  # soar_adamw_clip_multi_tensor_device: zero the gradients  # conv backward: weight-gradient addition at weight_grad_flush

# bytes of the static scratch behind soar_group_norm_backward_noalloc
# (SOAR_GN_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 4 << 20

TUNE_CHUNK = 1
TUNE_REVERSE = 2
TUNE_NT_STORE = 3
TUNE_BATCH_MB = 4
TUNE_STREAMS = 5
TUNE_NT_LOAD = 6
TUNE_CHUNK2 = 7
TUNE_PW_CHUNK = 8
TUNE_SMALL_UNIT = 9
TUNE_PW_SMALL = 10
TUNE_FOLD_MAX = 11
TUNE_PW_SPLITK = 12
TUNE_LOADS = 13
TUNE_PW_WG_WAVES = 14
TUNE_PW_WG_TARGET = 15
TUNE_PW_CBA_MIN = 16
TUNE_PW_CBA_BLOCKS = 17
TUNE_DW_CBA_MIN = 18
TUNE_NT_TAIL_MB = 19


class SoarUnavailable(RuntimeError):
    """The HIP library is not built or cannot be loaded."""


class SoarError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"soar status {code}: {message}")
        self.code = code
        self.message = message


_c = ctypes
_P = _c.c_void_p
_I64 = _c.c_int64
_SZ = _c.c_size_t

# name -> (restype, argtypes); every function include/soar_gn.h declares.
SIGNATURES = {
    "soar_last_error": (_c.c_char_p, []),
    "soar_is_device_available": (_c.c_int, []),
    "soar_gn_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "soar_gn_silu_forward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                        _c.c_float, _c.c_uint, _P, _SZ, _P]),
    "soar_gn_silu_backward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                         _I64, _I64, _c.c_uint, _P, _SZ, _P]),
    "soar_group_norm_forward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ,
                                           _c.c_float, _P]),
    "soar_group_norm_backward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ,
                                            _P]),
    "soar_group_norm_backward_noalloc": (_c.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _SZ,
                                                    _SZ, _SZ, _P]),
    "soar_silu_forward": (_c.c_int, [_P, _P, _SZ, _P]),
    "soar_silu_backward": (_c.c_int, [_P, _P, _P, _SZ, _P]),
    "soar_add_forward": (_c.c_int, [_P, _P, _P, _SZ, _P]),
    "soar_add_backward": (_c.c_int, [_P, _P, _P, _SZ, _P]),
    "soar_zero": (_c.c_int, [_P, _SZ, _P]),
    "soar_fill": (_c.c_int, [_P, _c.c_float, _SZ, _P]),
    "soar_conv2d_1x1_forward": (_c.c_int, [_P, _P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "soar_pw_conv_forward": (_c.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "soar_pw_conv_gn_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "soar_pw_conv_gn_silu_forward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                                _I64, _I64, _I64, _I64, _c.c_float, _c.c_uint,
                                                _P, _SZ, _P]),
    "soar_pw_conv_gn_silu_add_forward": (_c.c_int, [_P] * 11 + [_I64] * 5 +
                                         [_c.c_float, _c.c_uint, _P, _SZ, _P]),
    "soar_pw_conv_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "soar_pw_conv_backward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                         _c.c_uint, _P, _SZ, _P]),
    "soar_conv2d_1x1_backward": (_c.c_int, [_P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _P]),
    "soar_pw_cba_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "soar_pw_cba_backward": (_c.c_int, [_P] * 13 + [_I64] * 5 + [_c.c_uint, _P, _SZ, _P]),
    "soar_dw_conv_forward": (_c.c_int, [_P, _P, _P, _P] + [_I64] * 10 + [_P]),
    "soar_dw_conv_gn_workspace_bytes": (_SZ, [_I64] * 11),
    "soar_dw_conv_gn_silu_forward": (_c.c_int, [_P] * 10 + [_I64] * 11 +
                                     [_c.c_float, _c.c_uint, _P, _SZ, _P]),
    "soar_dw_conv_backward_workspace_bytes": (_SZ, [_I64] * 9),
    "soar_dw_conv_backward": (_c.c_int, [_P] * 6 + [_I64] * 10 + [_c.c_uint, _P, _SZ, _P]),
    "soar_dw_cba_backward_workspace_bytes": (_SZ, [_I64] * 11),
    "soar_dw_cba_backward": (_c.c_int, [_P] * 13 + [_I64] * 11 + [_c.c_uint, _P, _SZ, _P]),
    "soar_conv2d_dw_forward": (_c.c_int, [_P, _P, _P, _P] + [_SZ] * 9 + [_P]),
    "soar_conv2d_dw_backward": (_c.c_int, [_P] * 6 + [_SZ] * 9 + [_P]),
    "soar_arena_create": (_c.c_int, [_SZ, _SZ, _c.POINTER(_P)]),
    "soar_arena_alloc": (_c.c_int, [_P, _SZ, _c.POINTER(_P), _c.POINTER(_SZ)]),
    "soar_arena_freeze_static": (_c.c_int, [_P]),
    "soar_arena_reset_dynamic": (_c.c_int, [_P]),
    "soar_arena_info": (_c.c_int, [_P, _c.POINTER(_SZ), _c.POINTER(_SZ), _c.POINTER(_SZ),
                                   _c.POINTER(_P)]),
    "soar_arena_destroy": (_c.c_int, [_P]),
    "soar_memcpy_h2d": (_c.c_int, [_P, _P, _SZ, _P]),
    "soar_memcpy_d2h": (_c.c_int, [_P, _P, _SZ, _P]),
    "soar_memcpy_d2d": (_c.c_int, [_P, _P, _SZ, _P]),
    "soar_memcpy_async": (_c.c_int, [_P, _P, _SZ, _c.c_int, _P]),
    "soar_prof_enable": (_c.c_int, [_c.c_int]),
    "soar_weight_grad_flush": (_c.c_int, [_P]),
    "soar_weight_grad_pending": (_SZ, []),
    "soar_weight_grad_discard": (None, []),
    "soar_prof_summary": (_c.c_int, [_c.c_char_p, _SZ]),
    "soar_gn_tune": (_c.c_int, [_c.c_int, _I64]),
    "soar_gn_tune_get": (_I64, [_c.c_int]),
    # include/soar_ops.h
    "soar_conv2d_forward": (_c.c_int, [_P, _P, _P, _P] + [_SZ] * 11 + [_P]),
    "soar_conv2d_backward": (_c.c_int, [_P] * 6 + [_SZ] * 11 + [_P]),
    "soar_conv_forward": (_c.c_int, [_P, _P, _P, _P] + [_I64] * 12 + [_P]),
    "soar_conv_backward_workspace_bytes": (_SZ, [_I64] * 12),
    "soar_conv_backward": (_c.c_int, [_P] * 6 + [_I64] * 12 + [_c.c_uint, _P, _SZ, _P]),
    "soar_sigmoid_forward": (_c.c_int, [_P, _P, _SZ, _P]),
    "soar_sigmoid_backward": (_c.c_int, [_P, _P, _P, _SZ, _P]),
    "soar_mul_broadcast_forward": (_c.c_int, [_P, _P, _P, _SZ, _SZ, _P]),
    "soar_mul_broadcast_backward": (_c.c_int, [_P, _P, _P, _P, _P, _SZ, _SZ, _P]),
    "soar_convex_combination_forward": (_c.c_int, [_P, _P, _P, _P, _SZ, _P]),
    "soar_convex_combination_backward": (_c.c_int, [_P] * 7 + [_SZ, _P]),
    "soar_sigmoid_convex_forward": (_c.c_int, [_P, _P, _P, _P, _SZ, _P]),
    "soar_sigmoid_convex_backward_ex": (_c.c_int, [_P] * 7 + [_SZ, _c.c_uint, _P]),
    "soar_mul_sigmoid_broadcast_forward": (_c.c_int, [_P, _P, _P, _SZ, _SZ, _P]),
    "soar_mul_sigmoid_broadcast_backward_ex": (_c.c_int, [_P, _P, _P, _P, _P, _SZ, _SZ,
                                                          _c.c_uint, _P]),
    "soar_global_avg_pool_forward": (_c.c_int, [_P, _P, _SZ, _SZ, _P]),
    "soar_global_avg_pool_backward": (_c.c_int, [_P, _P, _SZ, _SZ, _P]),
    "soar_upsample_bilinear_forward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_upsample_bilinear_2x_forward": (_c.c_int, [_P, _P] + [_SZ] * 3 + [_P]),
    "soar_upsample_bilinear_backward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_upsample_bilinear_2x_backward": (_c.c_int, [_P, _P] + [_SZ] * 3 + [_P]),
    "soar_pixel_shuffle_forward": (_c.c_int, [_P, _P] + [_SZ] * 4 + [_P]),
    "soar_pixel_shuffle_backward": (_c.c_int, [_P, _P] + [_SZ] * 4 + [_P]),
    "soar_pad_spatial_forward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_pad_spatial_backward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_unpad_spatial_forward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_unpad_spatial_backward": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_P]),
    "soar_bce_with_logits_forward": (_c.c_int, [_P, _P, _c.c_float, _c.c_float, _SZ,
                                                _c.POINTER(_c.c_float), _P]),
    "soar_bce_with_logits_backward": (_c.c_int, [_P, _P, _P, _c.c_float, _c.c_float,
                                                 _c.c_float, _SZ, _P]),
    "soar_dice_loss_forward": (_c.c_int, [_P, _P, _c.c_float, _c.c_float,
                                          _c.POINTER(_c.c_float), _c.POINTER(_c.c_float),
                                          _c.POINTER(_c.c_float), _SZ,
                                          _c.POINTER(_c.c_float), _P]),
    "soar_dice_loss_backward": (_c.c_int, [_P, _P, _P] + [_c.c_float] * 6 + [_SZ, _P]),
    "soar_dice_bce_loss_forward": (_c.c_int, [_P, _P, _SZ] + [_c.c_float] * 5 +
                                   [_c.POINTER(_c.c_float), _P]),
    "soar_dice_bce_loss_backward": (_c.c_int, [_P, _P, _P] + [_c.c_float] * 9 + [_SZ, _P]),
    "soar_sigmoid_threshold": (_c.c_int, [_P, _P, _P, _SZ, _c.c_float, _P]),
    "soar_adamw_step": (_c.c_int, [_P, _P, _P, _P] + [_c.c_float] * 7 + [_SZ, _P]),
    "soar_adamw_step_multi_tensor": (_c.c_int, [_P, _P, _P, _P, _P, _c.c_int] +
                                     [_c.c_float] * 7 + [_P]),
    "soar_adamw_multi_tensor_device": (_c.c_int, [_P, _P, _P, _P, _P, _c.c_int] +
                                       [_c.c_float] * 7 + [_P]),
    "soar_multi_tensor_norm_workspace_bytes": (_SZ, []),
    "soar_multi_tensor_norm_sq_device": (_c.c_int, [_P, _P, _c.c_int, _P, _P, _SZ, _P]),
    "soar_multi_tensor_scale_device": (_c.c_int, [_P, _P, _c.c_int, _c.c_float, _P]),
    "soar_multi_tensor_fill_device": (_c.c_int, [_P, _P, _c.c_int, _c.c_float, _P]),
    "soar_adamw_multi_tensor_device_scalars": (_c.c_int, [_P, _P, _P, _P, _P, _c.c_int, _P] +
                                               [_c.c_float] * 4 + [_P]),
    "soar_multi_tensor_clip_device": (_c.c_int, [_P, _P, _c.c_int, _P, _c.c_float, _P]),
    "soar_multi_tensor_norm_sq_partials_device": (_c.c_int, [_P, _P, _c.c_int, _P, _SZ, _P]),
    "soar_adamw_clip_multi_tensor_device": (_c.c_int, [_P, _P, _P, _P, _P, _c.c_int, _P] +
                                            [_c.c_float] * 4 + [_P, _SZ, _c.c_float, _P,
                                                                _c.c_uint, _P]),
    "soar_dice_bce_loss_workspace_bytes": (_SZ, [_SZ]),
    "soar_dice_bce_loss_sums_device": (_c.c_int, [_P, _P, _SZ, _c.c_float, _P, _P, _SZ, _P]),
    "soar_dice_bce_loss_from_sums": (_c.c_int, [_P, _SZ] + [_c.c_float] * 4 + [_P]),
    "soar_dice_bce_loss_backward_device": (_c.c_int, [_P, _P, _P] + [_c.c_float] * 6 +
                                           [_P, _SZ, _c.c_uint, _P]),
    "soar_concat_channels_forward": (_c.c_int, [_P, _P, _c.c_int, _P, _I64, _I64, _P]),
    "soar_concat_channels_backward": (_c.c_int, [_P, _P, _P, _P, _c.c_int, _I64, _I64, _P]),
    "soar_sigmoid_backward_ex": (_c.c_int, [_P, _P, _P, _SZ, _c.c_uint, _P]),
    "soar_mul_broadcast_backward_ex": (_c.c_int, [_P, _P, _P, _P, _P, _SZ, _SZ, _c.c_uint, _P]),
    "soar_convex_combination_backward_ex": (_c.c_int, [_P] * 7 + [_SZ, _c.c_uint, _P]),
    "soar_global_avg_pool_backward_ex": (_c.c_int, [_P, _P, _SZ, _SZ, _c.c_uint, _P]),
    "soar_upsample_bilinear_backward_ex": (_c.c_int, [_P, _P] + [_SZ] * 5 + [_c.c_uint, _P]),
    "soar_pixel_shuffle_backward_ex": (_c.c_int, [_P, _P] + [_SZ] * 4 + [_c.c_uint, _P]),
    "soar_dice_bce_loss_backward_ex": (_c.c_int, [_P, _P, _P] + [_c.c_float] * 9 +
                                       [_SZ, _c.c_uint, _P]),
}

SYNTH_SIGNATURES = {
    "soar_synth_normal": (_c.c_int, [_P, _I64, _c.c_uint64, _c.c_uint32, _c.c_double,
                                     _c.c_double, _P]),
    "soar_synth_uniform": (_c.c_int, [_P, _I64, _c.c_uint64, _c.c_uint32, _c.c_double,
                                      _c.c_double, _P]),
    "soar_synth_stress": (_c.c_int, [_P, _I64, _c.c_uint64, _c.c_double, _c.c_double,
                                     _c.c_double, _c.c_double, _c.c_double, _P]),
    "soar_synth_copy": (_c.c_int, [_P, _P, _I64, _P]),
    "soar_synth_stream": (_c.c_int, [_c.c_int, _P, _P, _P, _I64, _P]),
    "soar_synth_planes": (_c.c_int, [_c.c_int, _P, _P, _I64, _I64, _P]),
    "soar_synth_stream_shape": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _I64,
                                           _c.c_int, _c.c_int, _P, _P, _P, _I64, _P]),
    "soar_synth_memcpy_d2d": (_c.c_int, [_P, _P, _I64, _P]),
}

_LIB = None
_SYNTH = None


OPS_HEADER_PATH = os.path.join(ROOT, "include", "soar_ops.h")


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of every function declared with SOAR_API in a header
    (include/soar_gn.h by default)."""
    with open(path) as f:
        text = f.read()
    return re.findall(r"SOAR_API\s+[^;(]*?\b(soar_\w+)\s*\(", text)


def _bind(path, signatures):
    if not os.path.exists(path):
        raise SoarUnavailable(
            f"{path} is not built; run `make -C soar.cpp_amd` or __graft_entry__.build()")
    try:
        handle = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise SoarUnavailable(f"cannot load {path}: {e}") from e
    for name, (res, args) in signatures.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def lib():
    """The loaded libsoar_gn.so (raises SoarUnavailable if absent)."""
    global _LIB
    if _LIB is None:
        _LIB = _bind(LIB_PATH, SIGNATURES)
    return _LIB


def synth_lib():
    global _SYNTH
    if _SYNTH is None:
        _SYNTH = _bind(SYNTH_PATH, SYNTH_SIGNATURES)
    return _SYNTH


def last_error() -> str:
    return lib().soar_last_error().decode()


def check(rc: int) -> int:
    if rc < 0:
        raise SoarError(rc, last_error())
    return rc


# ---- torch helpers ---------------------------------------------------------

def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _nchw(x):
    if x.dim() == 4:
        N, C, H, W = x.shape
        return N, C, H * W
    if x.dim() == 3:
        N, C, HW = x.shape
        return N, C, HW
    raise ValueError("expected [N,C,H,W] or [N,C,HW]")


def _check_tensor(t, name):
    import torch
    if t is None:
        return
    if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 device tensor")


def workspace_bytes(N, C, HW, G) -> int:
    return int(lib().soar_gn_workspace_bytes(N, C, HW, G))


def workspace(N, C, HW, G, device=None):
    import torch
    n = max(workspace_bytes(N, C, HW, G), 1)
    return torch.empty(n, dtype=torch.uint8, device=device or "cuda")


class Stats(tuple):
    """Saved statistics of a forward: (mean, rstd, mean_lo), float32[N*G]
    each; mean_lo is the fp32 rounding residual of the mean."""

    def __new__(cls, mean, rstd, mean_lo):
        return super().__new__(cls, (mean, rstd, mean_lo))

    mean = property(lambda s: s[0])
    rstd = property(lambda s: s[1])
    mean_lo = property(lambda s: s[2])


def gn_silu_forward(x, gamma, beta, G, eps=1e-5, silu=True, residual=False, y=None,
                    mean=None, rstd=None, mean_lo=None, keep_lo=True, ws=None, stream=None):
    """y = silu(group_norm(x)) [+ x] through soar_gn_silu_forward.

    Returns (y, Stats(mean, rstd, mean_lo)); mean_lo is None when keep_lo is
    False (the reference's fp32-mean-only saving)."""
    import torch
    N, C, HW = _nchw(x)
    for t, n in ((x, "x"), (gamma, "gamma"), (beta, "beta"), (y, "y"), (mean, "mean"),
                 (rstd, "rstd"), (mean_lo, "mean_lo")):
        _check_tensor(t, n)
    new = lambda: torch.empty(N * G, dtype=torch.float32, device=x.device)
    y = torch.empty_like(x) if y is None else y
    mean = new() if mean is None else mean
    rstd = new() if rstd is None else rstd
    if keep_lo and mean_lo is None:
        mean_lo = new()
    ws = workspace(N, C, HW, G, x.device) if ws is None else ws
    flags = (GN_SILU if silu else 0) | (GN_RESIDUAL if residual else 0)
    check(lib().soar_gn_silu_forward(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), _ptr(mean),
                                     _ptr(rstd), _ptr(mean_lo), N, C, HW, G, eps, flags,
                                     _ptr(ws), ws.numel(), _stream(stream)))
    return y, Stats(mean, rstd, mean_lo)


def gn_silu_backward(dy, x, gamma, beta, stats, G, silu=True, residual=False,
                     dx=None, dgamma=None, dbeta=None, want_dx=True, want_params=True,
                     accumulate_dx=False, ws=None, stream=None):
    """Backward through soar_gn_silu_backward; returns (dx, dgamma, dbeta).

    `stats` is the Stats of the forward (or a (mean, rstd[, mean_lo]) tuple).
    dgamma/dbeta are accumulated into (fresh zeros when not given)."""
    import torch
    mean, rstd = stats[0], stats[1]
    mean_lo = stats[2] if len(stats) > 2 else None
    N, C, HW = _nchw(x)
    for t, n in ((dy, "dy"), (x, "x"), (gamma, "gamma"), (beta, "beta"), (dx, "dx"),
                 (dgamma, "dgamma"), (dbeta, "dbeta")):
        _check_tensor(t, n)
    if want_dx and dx is None:
        dx = torch.empty_like(x) if not accumulate_dx else torch.zeros_like(x)
    if want_params:
        if dgamma is None:
            dgamma = torch.zeros(C, dtype=torch.float32, device=x.device)
        if dbeta is None:
            dbeta = torch.zeros(C, dtype=torch.float32, device=x.device)
    ws = workspace(N, C, HW, G, x.device) if ws is None else ws
    flags = ((GN_SILU if silu else 0) | (GN_RESIDUAL if residual else 0)
             | (GN_ACCUMULATE_DX if accumulate_dx else 0))
    check(lib().soar_gn_silu_backward(_ptr(dy), _ptr(x), _ptr(gamma), _ptr(beta),
                                      _ptr(mean), _ptr(rstd), _ptr(mean_lo),
                                      _ptr(dx) if want_dx else None,
                                      _ptr(dgamma) if want_params else None,
                                      _ptr(dbeta) if want_params else None,
                                      N, C, HW, G, flags, _ptr(ws), ws.numel(),
                                      _stream(stream)))
    return (dx if want_dx else None, dgamma if want_params else None,
            dbeta if want_params else None)


# ---- pointwise convolution ----------------------------------------------------

def conv1x1_forward(x, weight, bias=None, out=None, stream=None):
    """out[n] = weight @ x[n] + bias through soar_conv2d_1x1_forward, one call
    per sample (the reference operator's signature is per sample).

    x: [N, C_in, H, W], or one sample [C_in, H, W] / [C_in, HW]; weight:
    [C_out, C_in] (or [C_out, C_in, 1, 1]); bias: [C_out] or None."""
    import torch
    if x.dim() not in (2, 3, 4):
        raise ValueError("expected [N,C,H,W], [C,H,W] or [C,HW]")
    squeeze = x.dim() < 4
    xs = x.unsqueeze(0) if squeeze else x
    N, C_in = xs.shape[0], xs.shape[1]
    HW = 1
    for d in xs.shape[2:]:
        HW *= d
    w = weight.reshape(weight.shape[0], -1)
    C_out = w.shape[0]
    if w.shape[1] != C_in:
        raise ValueError("weight does not match the input channels")
    for t, n in ((xs, "x"), (w, "weight"), (bias, "bias"), (out, "out")):
        _check_tensor(t, n)
    if out is None:
        out = torch.empty((N, C_out) + tuple(xs.shape[2:]), dtype=torch.float32,
                          device=x.device)
    for n in range(N):
        check(lib().soar_conv2d_1x1_forward(_ptr(xs[n]), _ptr(w), _ptr(bias), _ptr(out[n]),
                                            C_in, C_out, HW, _stream(stream)))
    return out[0] if squeeze else out


def pw_conv_forward(x, weight, bias=None, z=None, stream=None):
    """z[n] = weight @ x[n] + bias for all samples in one soar_pw_conv_forward
    call.  x: [N, C_in, H, W] or [N, C_in, HW]; weight [C_out, C_in]."""
    import torch
    N, C_in, HW = _nchw(x)
    w = weight.reshape(weight.shape[0], -1)
    C_out = w.shape[0]
    if w.shape[1] != C_in:
        raise ValueError("weight does not match the input channels")
    for t, n in ((x, "x"), (w, "weight"), (bias, "bias"), (z, "z")):
        _check_tensor(t, n)
    if z is None:
        z = torch.empty((N, C_out) + tuple(x.shape[2:]), dtype=torch.float32, device=x.device)
    check(lib().soar_pw_conv_forward(_ptr(x), _ptr(w), _ptr(bias), _ptr(z), N, C_in, C_out, HW,
                                     _stream(stream)))
    return z


def pw_conv_gn_workspace_bytes(N, C_out, HW, G) -> int:
    return int(lib().soar_pw_conv_gn_workspace_bytes(N, C_out, HW, G))


def pw_conv_gn_silu_forward(x, weight, bias, gamma, beta, G, eps=1e-5, silu=True, z=None,
                            y=None, mean=None, rstd=None, mean_lo=None, ws=None,
                            stream=None, residual=None):
    """CBA forward of a pointwise conv through soar_pw_conv_gn_silu_forward
    (with `residual`: soar_pw_conv_gn_silu_add_forward, y += residual).

    Returns (z, y, Stats): z the convolution output (the GroupNorm input the
    backward needs), y = silu(group_norm(z)) (or group_norm(z))."""
    import torch
    N, C_in, HW = _nchw(x)
    w = weight.reshape(weight.shape[0], -1)
    C_out = w.shape[0]
    if w.shape[1] != C_in:
        raise ValueError("weight does not match the input channels")
    for t, n in ((x, "x"), (w, "weight"), (bias, "bias"), (gamma, "gamma"), (beta, "beta"),
                 (z, "z"), (y, "y"), (mean, "mean"), (rstd, "rstd"), (mean_lo, "mean_lo")):
        _check_tensor(t, n)
    shape = (N, C_out) + tuple(x.shape[2:])
    new = lambda: torch.empty(N * G, dtype=torch.float32, device=x.device)
    z = torch.empty(shape, dtype=torch.float32, device=x.device) if z is None else z
    y = torch.empty(shape, dtype=torch.float32, device=x.device) if y is None else y
    mean = new() if mean is None else mean
    rstd = new() if rstd is None else rstd
    mean_lo = new() if mean_lo is None else mean_lo
    if ws is None:
        ws = torch.empty(max(pw_conv_gn_workspace_bytes(N, C_out, HW, G), 1),
                         dtype=torch.uint8, device=x.device)
    if residual is not None:
        _check_tensor(residual, "residual")
        check(lib().soar_pw_conv_gn_silu_add_forward(
            _ptr(x), _ptr(w), _ptr(bias), _ptr(gamma), _ptr(beta), _ptr(residual), _ptr(z),
            _ptr(y), _ptr(mean), _ptr(rstd), _ptr(mean_lo), N, C_in, C_out, HW, G, eps,
            GN_SILU if silu else 0, _ptr(ws), ws.numel(), _stream(stream)))
        return z, y, Stats(mean, rstd, mean_lo)
    check(lib().soar_pw_conv_gn_silu_forward(
        _ptr(x), _ptr(w), _ptr(bias), _ptr(gamma), _ptr(beta), _ptr(z), _ptr(y), _ptr(mean),
        _ptr(rstd), _ptr(mean_lo), N, C_in, C_out, HW, G, eps, GN_SILU if silu else 0,
        _ptr(ws), ws.numel(), _stream(stream)))
    return z, y, Stats(mean, rstd, mean_lo)


def pw_conv_backward_workspace_bytes(N, C_in, C_out, HW) -> int:
    return int(lib().soar_pw_conv_backward_workspace_bytes(N, C_in, C_out, HW))


def pw_conv_backward(dz, x, weight, dx=None, dweight=None, dbias=None, want_dx=True,
                     want_dw=True, want_db=True, accumulate_dx=False, ws=None, stream=None,
                     defer_finish=False):
    """Backward of the pointwise conv through soar_pw_conv_backward; returns
    (dx, dweight, dbias).  dweight/dbias accumulate (fresh zeros when not
    given); dx is written, or added to with accumulate_dx.  defer_finish:
    dweight/dbias receive their sums at the next weight_grad_flush (keep ws
    alive until then)."""
    import torch
    N, C_out, HW = _nchw(dz)
    w = weight.reshape(weight.shape[0], -1)
    C_in = w.shape[1]
    for t, n in ((dz, "dz"), (x, "x"), (w, "weight"), (dx, "dx"), (dweight, "dweight"),
                 (dbias, "dbias")):
        _check_tensor(t, n)
    if want_dx and dx is None:
        shape = (N, C_in) + tuple(dz.shape[2:])
        dx = (torch.zeros if accumulate_dx else torch.empty)(shape, dtype=torch.float32,
                                                             device=dz.device)
    if want_dw and dweight is None:
        dweight = torch.zeros((C_out, C_in), dtype=torch.float32, device=dz.device)
    if want_db and dbias is None:
        dbias = torch.zeros(C_out, dtype=torch.float32, device=dz.device)
    if ws is None:
        ws = torch.empty(max(pw_conv_backward_workspace_bytes(N, C_in, C_out, HW), 1),
                         dtype=torch.uint8, device=dz.device)
    check(lib().soar_pw_conv_backward(
        _ptr(dz), _ptr(x), _ptr(w), _ptr(dx) if want_dx else None,
        _ptr(dweight) if want_dw else None, _ptr(dbias) if want_db else None, N, C_in, C_out,
        HW, (GN_ACCUMULATE_DX if accumulate_dx else 0) |
        (DEFER_WEIGHT_FINISH if defer_finish else 0), _ptr(ws), ws.numel(), _stream(stream)))
    return (dx if want_dx else None, dweight if want_dw else None, dbias if want_db else None)


def pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G) -> int:
    return int(lib().soar_pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G))


def pw_cba_backward(dy, z, x, weight, gamma, beta, stats, G, silu=True, dx=None, dweight=None,
                    dgamma=None, dbeta=None, want_dx=True, want_dw=True, want_params=True,
                    accumulate_dx=False, ws=None, stream=None, defer_finish=False):
    """Backward of a pointwise CBA block through soar_pw_cba_backward.

    z, stats: what pw_conv_gn_silu_forward returned; dy: the gradient at y.
    Returns (dx, dweight, dgamma, dbeta).  dweight/dgamma/dbeta accumulate
    (fresh zeros when not given); dx is written, or added to with
    accumulate_dx."""
    import torch
    N, C_out, HW = _nchw(z)
    w = weight.reshape(weight.shape[0], -1)
    C_in = w.shape[1]
    for t, n in ((dy, "dy"), (z, "z"), (x, "x"), (w, "weight"), (gamma, "gamma"),
                 (beta, "beta"), (dx, "dx"), (dweight, "dweight"), (dgamma, "dgamma"),
                 (dbeta, "dbeta")):
        _check_tensor(t, n)
    dev = z.device
    if want_dx and dx is None:
        shape = (N, C_in) + tuple(z.shape[2:])
        dx = (torch.zeros if accumulate_dx else torch.empty)(shape, dtype=torch.float32,
                                                             device=dev)
    if want_dw and dweight is None:
        dweight = torch.zeros((C_out, C_in), dtype=torch.float32, device=dev)
    if want_params and dgamma is None:
        dgamma = torch.zeros(C_out, dtype=torch.float32, device=dev)
    if want_params and dbeta is None:
        dbeta = torch.zeros(C_out, dtype=torch.float32, device=dev)
    if ws is None:
        ws = torch.empty(max(pw_cba_backward_workspace_bytes(N, C_in, C_out, HW, G), 1),
                         dtype=torch.uint8, device=dev)
    flags = ((GN_SILU if silu else 0) | (GN_ACCUMULATE_DX if accumulate_dx else 0) |
             (DEFER_WEIGHT_FINISH if defer_finish else 0))
    check(lib().soar_pw_cba_backward(
        _ptr(dy), _ptr(z), _ptr(x), _ptr(w), _ptr(gamma), _ptr(beta), _ptr(stats.mean),
        _ptr(stats.rstd), _ptr(stats.mean_lo), _ptr(dx) if want_dx else None,
        _ptr(dweight) if want_dw else None, _ptr(dgamma) if want_params else None,
        _ptr(dbeta) if want_params else None, N, C_in, C_out, HW, G, flags, _ptr(ws),
        ws.numel(), _stream(stream)))
    return (dx if want_dx else None, dweight if want_dw else None,
            dgamma if want_params else None, dbeta if want_params else None)


# ---- depthwise convolution -------------------------------------------------------

def conv_out_size(H, K, pad, stride, dil):
    """Conv2d's output size (src/nn/layers.cpp:330-332)."""
    return (H + 2 * pad - (dil * (K - 1) + 1)) // stride + 1


def dw_conv_forward(x, weight, bias, pad, stride=1, dil=1, y=None, stream=None):
    """Depthwise conv through soar_dw_conv_forward.  x [N,C,H,W], weight
    [C,K,K] (or [C,1,K,K]), bias [C] or None; returns y [N,C,Ho,Wo]."""
    import torch
    N, C, H, W = x.shape
    K = weight.shape[-1]
    Ho, Wo = conv_out_size(H, K, pad, stride, dil), conv_out_size(W, K, pad, stride, dil)
    for t, n in ((x, "x"), (weight, "weight"), (bias, "bias"), (y, "y")):
        _check_tensor(t, n)
    if y is None:
        y = torch.empty((N, C, Ho, Wo), dtype=torch.float32, device=x.device)
    check(lib().soar_dw_conv_forward(_ptr(x), _ptr(weight), _ptr(bias), _ptr(y), N, C, H, W,
                                     Ho, Wo, K, pad, stride, dil, _stream(stream)))
    return y


def dw_conv_gn_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride, dil, G) -> int:
    return int(lib().soar_dw_conv_gn_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride, dil, G))


def dw_conv_gn_silu_forward(x, weight, bias, gamma, beta, G, pad, stride=1, dil=1, eps=1e-5,
                            silu=True, z=None, y=None, mean=None, rstd=None, mean_lo=None,
                            ws=None, stream=None):
    """CBA forward of a depthwise conv through soar_dw_conv_gn_silu_forward.
    x [N,C,H,W], weight [C,K,K]; returns (z, y, Stats): z the convolution
    output (the GroupNorm input the backward needs), y = silu(group_norm(z))
    (or group_norm(z))."""
    import torch
    N, C, H, W = x.shape
    K = weight.shape[-1]
    Ho, Wo = conv_out_size(H, K, pad, stride, dil), conv_out_size(W, K, pad, stride, dil)
    for t, n in ((x, "x"), (weight, "weight"), (bias, "bias"), (gamma, "gamma"),
                 (beta, "beta"), (z, "z"), (y, "y"), (mean, "mean"), (rstd, "rstd"),
                 (mean_lo, "mean_lo")):
        _check_tensor(t, n)
    shape = (N, C, Ho, Wo)
    new = lambda: torch.empty(N * G, dtype=torch.float32, device=x.device)
    z = torch.empty(shape, dtype=torch.float32, device=x.device) if z is None else z
    y = torch.empty(shape, dtype=torch.float32, device=x.device) if y is None else y
    mean = new() if mean is None else mean
    rstd = new() if rstd is None else rstd
    mean_lo = new() if mean_lo is None else mean_lo
    if ws is None:
        ws = torch.empty(max(dw_conv_gn_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride, dil,
                                                        G), 1),
                         dtype=torch.uint8, device=x.device)
    check(lib().soar_dw_conv_gn_silu_forward(
        _ptr(x), _ptr(weight), _ptr(bias), _ptr(gamma), _ptr(beta), _ptr(z), _ptr(y),
        _ptr(mean), _ptr(rstd), _ptr(mean_lo), N, C, H, W, Ho, Wo, K, pad, stride, dil, G, eps,
        GN_SILU if silu else 0, _ptr(ws), ws.numel(), _stream(stream)))
    return z, y, Stats(mean, rstd, mean_lo)


def dw_conv_backward(dy, x, weight, pad, stride=1, dil=1, dx=None, dweight=None, dbias=None,
                     want_dx=True, want_dw=True, want_db=True, accumulate_dx=False, ws=None,
                     stream=None, defer_finish=False):
    """Backward through soar_dw_conv_backward; returns (dx, dweight, dbias).
    dweight/dbias accumulate (fresh zeros when not given)."""
    import torch
    N, C, H, W = x.shape
    K = weight.shape[-1]
    Ho, Wo = dy.shape[2], dy.shape[3]
    for t, n in ((dy, "dy"), (x, "x"), (weight, "weight"), (dx, "dx"), (dweight, "dweight"),
                 (dbias, "dbias")):
        _check_tensor(t, n)
    if want_dx and dx is None:
        dx = (torch.zeros if accumulate_dx else torch.empty)((N, C, H, W), dtype=torch.float32,
                                                             device=x.device)
    if want_dw and dweight is None:
        dweight = torch.zeros((C, K, K), dtype=torch.float32, device=x.device)
    if want_db and dbias is None:
        dbias = torch.zeros(C, dtype=torch.float32, device=x.device)
    if ws is None:
        n = int(lib().soar_dw_conv_backward_workspace_bytes(N, C, H, W, Ho, Wo, K, stride, dil))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=x.device)
    check(lib().soar_dw_conv_backward(
        _ptr(dy), _ptr(x), _ptr(weight), _ptr(dx) if want_dx else None,
        _ptr(dweight) if want_dw else None, _ptr(dbias) if want_db else None, N, C, H, W, Ho,
        Wo, K, pad, stride, dil, (GN_ACCUMULATE_DX if accumulate_dx else 0) |
        (DEFER_WEIGHT_FINISH if defer_finish else 0), _ptr(ws), ws.numel(), _stream(stream)))
    return (dx if want_dx else None, dweight if want_dw else None, dbias if want_db else None)


def dw_cba_backward_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride, dil, G) -> int:
    return int(lib().soar_dw_cba_backward_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride,
                                                          dil, G))


def dw_cba_backward(dy, z, x, weight, gamma, beta, stats, G, pad, stride=1, dil=1, silu=True,
                    dx=None, dweight=None, dgamma=None, dbeta=None, want_dx=True, want_dw=True,
                    want_params=True, accumulate_dx=False, ws=None, stream=None,
                    defer_finish=False):
    """Backward of a depthwise CBA block through soar_dw_cba_backward.

    z: the convolution output (the GroupNorm input), stats: its GroupNorm
    forward's Stats, dy: the gradient at the block's output.  Returns
    (dx, dweight, dgamma, dbeta); dweight/dgamma/dbeta accumulate (fresh
    zeros when not given); dx is written, or added to with accumulate_dx."""
    import torch
    N, C, H, W = x.shape
    Ho, Wo = z.shape[2], z.shape[3]
    K = weight.shape[-1]
    for t, n in ((dy, "dy"), (z, "z"), (x, "x"), (weight, "weight"), (gamma, "gamma"),
                 (beta, "beta"), (dx, "dx"), (dweight, "dweight"), (dgamma, "dgamma"),
                 (dbeta, "dbeta")):
        _check_tensor(t, n)
    dev = x.device
    if want_dx and dx is None:
        dx = (torch.zeros if accumulate_dx else torch.empty)((N, C, H, W), dtype=torch.float32,
                                                             device=dev)
    if want_dw and dweight is None:
        dweight = torch.zeros((C, K, K), dtype=torch.float32, device=dev)
    if want_params and dgamma is None:
        dgamma = torch.zeros(C, dtype=torch.float32, device=dev)
    if want_params and dbeta is None:
        dbeta = torch.zeros(C, dtype=torch.float32, device=dev)
    if ws is None:
        n = dw_cba_backward_workspace_bytes(N, C, H, W, Ho, Wo, K, pad, stride, dil, G)
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
    flags = ((GN_SILU if silu else 0) | (GN_ACCUMULATE_DX if accumulate_dx else 0) |
             (DEFER_WEIGHT_FINISH if defer_finish else 0))
    check(lib().soar_dw_cba_backward(
        _ptr(dy), _ptr(z), _ptr(x), _ptr(weight), _ptr(gamma), _ptr(beta), _ptr(stats.mean),
        _ptr(stats.rstd), _ptr(stats.mean_lo), _ptr(dx) if want_dx else None,
        _ptr(dweight) if want_dw else None, _ptr(dgamma) if want_params else None,
        _ptr(dbeta) if want_params else None, N, C, H, W, Ho, Wo, K, pad, stride, dil, G, flags,
        _ptr(ws), ws.numel(), _stream(stream)))
    return (dx if want_dx else None, dweight if want_dw else None,
            dgamma if want_params else None, dbeta if want_params else None)


def weight_grad_flush(stream=None):
    """Runs the weight-gradient finishes this thread's backward calls left
    pending (defer_finish=True) in one launch, on the stream they were
    queued on (`stream` must be it)."""
    check(lib().soar_weight_grad_flush(_stream(stream)))


def weight_grad_pending() -> int:
    return int(lib().soar_weight_grad_pending())


def weight_grad_discard():
    """Drops this thread's pending weight-gradient finishes unrun."""
    lib().soar_weight_grad_discard()


def prof_enable(on: bool = True):
    check(lib().soar_prof_enable(1 if on else 0))


def prof_summary() -> list[dict]:
    buf = ctypes.create_string_buffer(1 << 16)
    check(lib().soar_prof_summary(buf, len(buf)))
    return json.loads(buf.value.decode() or "[]")


def tune(key: int, value: int):
    check(lib().soar_gn_tune(key, value))


def tune_get(key: int) -> int:
    return int(lib().soar_gn_tune_get(key))


# ---- synthetic inputs (libsoar_synth.so) ------------------------------------

def synth_normal(t, seed, stream_id, mean=0.0, std=1.0, stream=None):
    rc = synth_lib().soar_synth_normal(_ptr(t), t.numel(), seed, stream_id, mean, std,
                                       _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_normal failed")
    return t


def synth_uniform(t, seed, stream_id, lo, hi, stream=None):
    rc = synth_lib().soar_synth_uniform(_ptr(t), t.numel(), seed, stream_id, lo, hi,
                                        _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_uniform failed")
    return t


def synth_stress(t, seed, center=1e3, std=1e-2, p=1e-3, out_mean=0.0, out_std=50.0,
                 stream=None):
    rc = synth_lib().soar_synth_stress(_ptr(t), t.numel(), seed, center, std, p, out_mean,
                                       out_std, _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_stress failed")
    return t


# kinds of synth_stream: name -> (kind, tensor passes per launch)
STREAM_KINDS = {"read": (0, 1), "copy": (1, 2), "2r1w": (2, 3), "2r": (3, 2)}


def synth_stream_shape(kind, a, b, out, threads, loads, chunk=None, grid=None, ntl=False,
                       nts=True, stream=None):
    """A streaming pattern (as synth_stream) in another launch shape
    (soar_synth_stream_shape): `chunk` floats per block, or a persistent
    grid of `grid` blocks; `loads` float4 loads per thread and tensor in
    flight; non-temporal loads / stores."""
    k = STREAM_KINDS[kind][0]
    for t in (a, b, out):
        if t is not None and t.numel() != a.numel():
            raise ValueError("synth_stream_shape buffers must have equal sizes")
    persistent = grid is not None
    rc = synth_lib().soar_synth_stream_shape(k, int(persistent), threads, loads,
                                             grid if persistent else chunk, int(ntl), int(nts),
                                             _ptr(a), _ptr(b), _ptr(out), a.numel(),
                                             _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_stream_shape failed")


def synth_memcpy_d2d(dst, src, stream=None):
    """dst = src through the runtime's device-to-device hipMemcpyAsync."""
    if dst.numel() != src.numel():
        raise ValueError("synth_memcpy_d2d buffers must have equal sizes")
    rc = synth_lib().soar_synth_memcpy_d2d(_ptr(dst), _ptr(src), src.numel(), _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_memcpy_d2d failed")


def synth_stream(kind, a, b, out, stream=None):
    """One launch of a streaming-ceiling kernel (soar_synth_stream): kind
    "read" reads a, "copy" copies a to out, "2r1w" writes out = a + b, "2r"
    reads a and b.  Buffers: equal-sized contiguous float32."""
    k = STREAM_KINDS[kind][0]
    for t in (a, b, out):
        if t is not None and t.numel() != a.numel():
            raise ValueError("synth_stream buffers must have equal sizes")
    rc = synth_lib().soar_synth_stream(k, _ptr(a), _ptr(b), _ptr(out), a.numel(),
                                       _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_stream failed")


def synth_planes(write, a, out, plane_floats, stride_floats, stream=None):
    """One launch of the 64-plane access pattern of the pointwise
    convolution (soar_synth_planes); a and out hold 64 * stride_floats
    floats."""
    for t in (a, out):
        if t.numel() < 64 * stride_floats:
            raise ValueError("synth_planes buffers must hold 64 planes at the stride")
    rc = synth_lib().soar_synth_planes(1 if write else 0, _ptr(a), _ptr(out), plane_floats,
                                       stride_floats, _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_planes failed")


def synth_copy(src, dst, stream=None):
    rc = synth_lib().soar_synth_copy(_ptr(src), _ptr(dst), src.numel(), _stream(stream))
    if rc:
        raise SoarError(rc, "soar_synth_copy failed")
    return dst
