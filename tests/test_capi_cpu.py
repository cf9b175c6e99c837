"""The C-ABI library on the CPU: it loads, exports every symbol the header
declares, and validates arguments without touching a GPU."""
import ctypes

import pytest

import soar_gn


@pytest.fixture(scope="module")
def L():
    return soar_gn.lib()


def test_exports_every_header_symbol(L):
    names = soar_gn.header_symbols() + soar_gn.header_symbols(soar_gn.OPS_HEADER_PATH)
    assert len(names) >= 60
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the binding declares exactly those
    assert set(names) == set(soar_gn.SIGNATURES)


def test_ops_validate_on_the_host(L):
    """Shape errors of the model operators are caught before any device
    call (so they hold without a GPU)."""
    # output size that does not match the input / kernel / stride
    assert L.soar_conv2d_forward(None, None, None, None, 1, 16, 64, 64, 31, 32, 3, 1, 2, 1,
                                 1, None) == soar_gn.SOAR_EINVAL
    assert b"does not match" in L.soar_last_error()
    # channels not divisible by groups
    assert L.soar_conv_forward(None, None, None, None, 1, 6, 4, 8, 8, 8, 8, 3, 1, 1, 1, 4,
                               None) == soar_gn.SOAR_EINVAL
    # pixel shuffle needs C_in divisible by r*r
    assert L.soar_pixel_shuffle_forward(None, None, 6, 4, 4, 2, None) == soar_gn.SOAR_EINVAL
    # crop larger than the padded plane
    assert L.soar_unpad_spatial_forward(None, None, 1, 4, 4, 5, 4, None) == soar_gn.SOAR_EINVAL
    # the _ex backward entry points know one flag (add instead of write)
    assert L.soar_sigmoid_backward_ex(None, None, None, 4, 1, None) == soar_gn.SOAR_EINVAL
    assert b"unsupported flags" in L.soar_last_error()
    assert L.soar_convex_combination_backward_ex(None, None, None, None, None, None, None, 4,
                                                 8, None) == soar_gn.SOAR_EINVAL
    # concatenation: 1..16 pieces, non-negative channel counts, one flag
    ch = (ctypes.c_int64 * 17)(*([1] * 17))
    ptrs = (ctypes.c_void_p * 17)()
    assert L.soar_concat_channels_forward(ptrs, ch, 0, None, 1, 4, None) == soar_gn.SOAR_EINVAL
    assert L.soar_concat_channels_forward(ptrs, ch, 17, None, 1, 4, None) == soar_gn.SOAR_EINVAL
    neg = (ctypes.c_int64 * 2)(3, -1)
    assert L.soar_concat_channels_forward(ptrs, neg, 2, None, 1, 4, None) == soar_gn.SOAR_EINVAL
    fl = (ctypes.c_uint * 2)(0, 1)
    assert L.soar_concat_channels_backward(None, ptrs, ch, fl, 2, 1, 4,
                                           None) == soar_gn.SOAR_EINVAL
    assert b"unsupported flags" in L.soar_last_error()
    # resize: plane sides must stay below 2^31 (the tap arithmetic is 32-bit)
    assert L.soar_upsample_bilinear_forward(None, None, 1, 1, 1 << 31, 2, 2,
                                            None) == soar_gn.SOAR_EINVAL
    assert b"2^31" in L.soar_last_error()
    assert L.soar_upsample_bilinear_backward(None, None, 1, 2, 2, 1 << 31, 1,
                                             None) == soar_gn.SOAR_EINVAL
    # conv workspace is pure host arithmetic: one fp64 partial per (weight
    # tap or bias, position chunk).  Grouped (or K > 3, or C_out % 4) convs:
    # chunks of 1024..16384 positions, sized for about 2048 blocks over the
    # 16 (co, q) rows: 1024 here
    assert L.soar_conv_backward_workspace_bytes(1, 2, 16, 64, 64, 32, 32, 3, 1, 2, 1, 2) == \
        16 * 10 * 1 * 8
    # dense few-channel convs (the stem): chunks of at least 512 positions,
    # about 2048 blocks over the 4-channel wave groups: 2 and 64 chunks
    assert L.soar_conv_backward_workspace_bytes(1, 1, 16, 64, 64, 32, 32, 3, 1, 2, 1, 1) == \
        16 * 10 * 2 * 8
    assert L.soar_conv_backward_workspace_bytes(2, 1, 16, 256, 256, 128, 128, 3, 1, 2, 1, 1) == \
        16 * 10 * 64 * 8
    # one row (co, q) wants 2048 chunks, capped below by 1024 positions
    assert L.soar_conv_backward_workspace_bytes(1, 1, 1, 1024, 1024, 512, 512, 3, 1, 2, 1, 1) == \
        1 * 10 * 256 * 8
    assert L.soar_multi_tensor_norm_workspace_bytes() == (512 + 1) * 8


def test_synth_library_exports(L):
    S = soar_gn.synth_lib()
    for n in soar_gn.SYNTH_SIGNATURES:
        assert hasattr(S, n)


def test_workspace_bytes_is_host_arithmetic(L):
    # cfg 3: 64 planes x 512 chunks of 8192 floats -> 32768 partials of 16 B
    assert soar_gn.tune_get(soar_gn.TUNE_CHUNK) == 8192
    # plus 64 plane sums of 16 B, 16 unit sums of 16 B, 16 mean residuals
    # of 4 B and 32768 chunk sums of x - mean of 8 B (the backward's mean
    # residual recovery), each region 256-byte aligned.
    assert soar_gn.workspace_bytes(1, 64, 2048 * 2048, 16) == \
        32768 * 16 + 1024 + 2 * 256 + 32768 * 8
    # small planes get one block each (chunk clipped to the plane)
    assert soar_gn.workspace_bytes(2, 6, 10, 3) == 5 * 256
    assert soar_gn.workspace_bytes(0, 6, 10, 3) == 0
    assert soar_gn.workspace_bytes(1, 6, 10, 4) == 0  # C % G != 0


def _fwd(L, N, C, HW, G, flags=1, eps=1e-5):
    return L.soar_gn_silu_forward(None, None, None, None, None, None, None, N, C, HW, G, eps,
                                  flags, None, 0, None)


def test_forward_validation_without_gpu(L):
    assert _fwd(L, 1, 6, 16, 4) == soar_gn.SOAR_EINVAL
    assert "divisible" in soar_gn.last_error()
    assert _fwd(L, 1, 6, 16, 0) == soar_gn.SOAR_EINVAL
    assert _fwd(L, -1, 6, 16, 3) == soar_gn.SOAR_EINVAL
    assert _fwd(L, 1, 6, 16, 3, flags=4) == soar_gn.SOAR_EINVAL  # ACCUMULATE_DX is bwd-only
    assert _fwd(L, 1, 6, 16, 3, eps=-1.0) == soar_gn.SOAR_EINVAL
    assert _fwd(L, 1 << 40, 1 << 20, 1 << 20, 1) == soar_gn.SOAR_EINVAL  # overflow
    # empty tensors are a successful no-op, as the reference returns early
    assert _fwd(L, 0, 6, 16, 3) == soar_gn.SOAR_OK
    assert _fwd(L, 1, 6, 0, 3) == soar_gn.SOAR_OK
    assert soar_gn.last_error() == ""


def test_no_device_is_reported_not_faulted(L):
    if L.soar_is_device_available():
        pytest.skip("a device is visible")
    assert _fwd(L, 1, 6, 16, 3) == soar_gn.SOAR_ENODEV
    p = ctypes.c_void_p()
    assert L.soar_arena_create(1 << 20, 256, ctypes.byref(p)) == soar_gn.SOAR_ENODEV
    assert L.soar_silu_forward(None, None, 16, None) == soar_gn.SOAR_ENODEV


def test_backward_validation_without_gpu(L):
    f = L.soar_gn_silu_backward
    dummy = ctypes.c_void_p(0x1000)
    # dgamma without dbeta is a valid request (each parameter gradient is
    # optional, normalization_kernels.cu:142-152): it passes validation and
    # reaches the device check
    rc = f(None, None, None, None, None, None, None, None, dummy, None, 1, 6, 16, 3, 1, None, 0,
           None)
    if not L.soar_is_device_available():
        assert rc == soar_gn.SOAR_ENODEV
    rc = f(None, None, None, None, None, None, None, None, None, dummy, 1, 6, 16, 3, 1, None, 0,
           None)
    if not L.soar_is_device_available():
        assert rc == soar_gn.SOAR_ENODEV
    rc = f(None, None, None, None, None, None, None, None, None, None, 1, 6, 16, 3, 8, None, 0,
           None)
    assert rc == soar_gn.SOAR_EINVAL  # unknown flag
    # nothing requested -> no-op
    rc = f(None, None, None, None, None, None, None, None, None, None, 1, 6, 16, 3, 1, None, 0,
           None)
    assert rc == soar_gn.SOAR_OK


def test_tuning_knobs(L):
    old = soar_gn.tune_get(soar_gn.TUNE_CHUNK)
    assert L.soar_gn_tune(soar_gn.TUNE_CHUNK, 1000) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_REVERSE, 2) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(99, 1) == soar_gn.SOAR_EINVAL
    soar_gn.tune(soar_gn.TUNE_CHUNK, 4096)
    assert soar_gn.workspace_bytes(1, 64, 2048 * 2048, 16) == \
        65536 * 16 + 1024 + 2 * 256 + 65536 * 8
    assert L.soar_gn_tune(soar_gn.TUNE_BATCH_MB, -1) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_CHUNK2, 1536) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_STREAMS, 3) == soar_gn.SOAR_EINVAL
    # non-temporal loads: a 2-bit mask (second passes, first passes)
    for bad in (-1, 4):
        assert L.soar_gn_tune(soar_gn.TUNE_NT_LOAD, bad) == soar_gn.SOAR_EINVAL
    nt = soar_gn.tune_get(soar_gn.TUNE_NT_LOAD)
    for v in (0, 1, 2, 3):
        soar_gn.tune(soar_gn.TUNE_NT_LOAD, v)
        assert soar_gn.tune_get(soar_gn.TUNE_NT_LOAD) == v
    soar_gn.tune(soar_gn.TUNE_NT_LOAD, nt)
    assert nt == 3 and soar_gn.tune_get(soar_gn.TUNE_NT_TAIL_MB) == 256
    for bad in (-1, (1 << 20) + 1):
        assert L.soar_gn_tune(soar_gn.TUNE_NT_TAIL_MB, bad) == soar_gn.SOAR_EINVAL
    assert soar_gn.tune_get(soar_gn.TUNE_CHUNK2) == 4096
    assert soar_gn.tune_get(soar_gn.TUNE_BATCH_MB) == 0
    soar_gn.tune(soar_gn.TUNE_CHUNK, old)
    assert soar_gn.tune_get(soar_gn.TUNE_CHUNK) == old


def test_prof_summary_empty(L):
    soar_gn.prof_enable(False)
    assert soar_gn.prof_summary() == []


def test_reference_signature_validation(L):
    rc = L.soar_group_norm_forward(None, None, None, None, None, None, 4, 6, 16, 1e-5, None)
    assert rc == soar_gn.SOAR_EINVAL
    rc = L.soar_group_norm_forward(None, None, None, None, None, None, 3, 6, 0, 1e-5, None)
    assert rc == soar_gn.SOAR_OK
    assert L.soar_add_backward(None, None, None, 10, None) == soar_gn.SOAR_OK
    assert L.soar_fill(None, 1.0, 0, None) == soar_gn.SOAR_OK


# ---- pointwise convolution -------------------------------------------------------

def _pw(L, N, C_in, C_out, HW, G, flags=1, eps=1e-5):
    return L.soar_pw_conv_gn_silu_forward(None, None, None, None, None, None, None, None, None,
                                          None, N, C_in, C_out, HW, G, eps, flags, None, 0,
                                          None)


def test_pw_conv_workspace_bytes(L):
    assert soar_gn.tune_get(soar_gn.TUNE_PW_CHUNK) == 1024
    # 64 output planes x 4096 chunks of 1024 pixels -> 262144 partials of
    # 16 B, then plane sums, unit sums, mean residuals and the 8-byte chunk
    # sums of the backward's mean residual recovery (256-byte aligned)
    assert soar_gn.pw_conv_gn_workspace_bytes(1, 64, 2048 * 2048, 16) == (
        262144 * 16 + 1024 + 2 * 256 + 262144 * 8)
    # a plane shorter than the chunk is one chunk; a grid this small (2
    # tiles) may split K over up to 8 blocks, so 8 fp32 slices of z follow
    assert soar_gn.pw_conv_gn_workspace_bytes(2, 8, 100, 2) == (
        5 * 256 + 8 * 2 * 8 * 100 * 4)
    soar_gn.tune(soar_gn.TUNE_PW_SPLITK, 1)
    try:
        assert soar_gn.pw_conv_gn_workspace_bytes(2, 8, 100, 2) == 5 * 256
    finally:
        soar_gn.tune(soar_gn.TUNE_PW_SPLITK, 8)
    assert L.soar_gn_tune(soar_gn.TUNE_PW_SPLITK, 0) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_PW_SPLITK, 9) == soar_gn.SOAR_EINVAL
    assert soar_gn.tune_get(soar_gn.TUNE_PW_SPLITK) == 8
    assert soar_gn.pw_conv_gn_workspace_bytes(1, 6, 10, 4) == 0  # C_out % G != 0
    assert soar_gn.pw_conv_gn_workspace_bytes(0, 6, 10, 3) == 0


def test_pw_conv_validation_without_gpu(L):
    assert _pw(L, 1, 8, 6, 16, 4) == soar_gn.SOAR_EINVAL
    assert "divisible" in soar_gn.last_error()
    assert _pw(L, -1, 8, 6, 16, 3) == soar_gn.SOAR_EINVAL
    assert _pw(L, 1, -8, 6, 16, 3) == soar_gn.SOAR_EINVAL
    assert _pw(L, 1, 8, 6, 16, 3, flags=2) == soar_gn.SOAR_EINVAL  # residual is not fused here
    assert "flags" in soar_gn.last_error()
    assert _pw(L, 1, 8, 6, 16, 3, eps=-1.0) == soar_gn.SOAR_EINVAL
    assert _pw(L, 1, 0, 6, 16, 3) == soar_gn.SOAR_EINVAL  # no input channels
    assert _pw(L, 1, 1 << 42, 1 << 20, 1 << 20, 1) == soar_gn.SOAR_EINVAL  # overflow
    # planes too long for the kernel's 32-bit in-sample offsets
    assert _pw(L, 1, 8, 6, 1 << 28, 3) == soar_gn.SOAR_EINVAL
    assert "32-bit" in soar_gn.last_error()
    assert _pw(L, 0, 8, 6, 16, 3) == soar_gn.SOAR_OK  # empty
    assert _pw(L, 1, 8, 6, 0, 3) == soar_gn.SOAR_OK
    f = L.soar_conv2d_1x1_forward
    assert f(None, None, None, None, 8, 6, 0, None) == soar_gn.SOAR_OK
    assert f(None, None, None, None, 0, 6, 16, None) == soar_gn.SOAR_EINVAL
    assert f(None, None, None, None, 8, 6, 1 << 28, None) == soar_gn.SOAR_EINVAL


def _dwf(L, N, C, H, W, K, G, flags=1, eps=1e-5, stride=1, dil=1):
    pad = dil * (K - 1) // 2
    Ho = (H + 2 * pad - dil * (K - 1) - 1) // stride + 1
    Wo = (W + 2 * pad - dil * (K - 1) - 1) // stride + 1
    return L.soar_dw_conv_gn_silu_forward(None, None, None, None, None, None, None, None, None,
                                          None, N, C, H, W, Ho, Wo, K, pad, stride, dil, G, eps,
                                          flags, None, 0, None)


def test_dw_conv_gn_workspace_bytes(L):
    al = lambda b: (b + 255) // 256 * 256
    gn = soar_gn.workspace_bytes(1, 64, 2048 * 2048, 16)
    # k7 at 64 x 2048^2: tile groups of 16 tiles of 32 x 64 outputs, 4 x 32
    # groups per plane -> 64 x 128 partials of 16 B after the GroupNorm part
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 64, 2048, 2048, 2048, 2048, 7, 3, 1, 1, 16) \
        == al(gn) + 64 * 128 * 16
    # k5 and k3 at dilation 1 run two output rows per thread (64-row tiles),
    # k5 in groups of 8 tiles (4 x 32 per plane), k3 of 4 (8 x 32 per plane)
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 64, 2048, 2048, 2048, 2048, 5, 2, 1, 1, 16) \
        == al(gn) + 64 * 128 * 16
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 64, 2048, 2048, 2048, 2048, 3, 1, 1, 1, 16) \
        == al(gn) + 64 * 256 * 16
    # units small enough for the one-launch GroupNorm: its workspace alone
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 8, 32, 32, 32, 32, 3, 1, 1, 1, 2) == \
        al(soar_gn.workspace_bytes(1, 8, 32 * 32, 2))
    # no tiled kernel (K = 9): the GroupNorm workspace alone
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 8, 128, 128, 128, 128, 9, 4, 1, 1, 2) == \
        al(soar_gn.workspace_bytes(1, 8, 128 * 128, 2))
    assert soar_gn.dw_conv_gn_workspace_bytes(1, 6, 64, 64, 64, 64, 3, 1, 1, 1, 4) == 0  # C % G
    assert soar_gn.dw_conv_gn_workspace_bytes(0, 8, 64, 64, 64, 64, 3, 1, 1, 1, 2) == 0


def test_dw_conv_gn_validation_without_gpu(L):
    assert _dwf(L, 1, 6, 64, 64, 3, 4) == soar_gn.SOAR_EINVAL
    assert "divisible" in soar_gn.last_error()
    assert _dwf(L, 1, 8, 64, 64, 3, 2, flags=2) == soar_gn.SOAR_EINVAL  # residual not fused
    assert "flags" in soar_gn.last_error()
    assert _dwf(L, 1, 8, 64, 64, 3, 2, eps=-1.0) == soar_gn.SOAR_EINVAL
    assert _dwf(L, 1, 8, 64, 64, 0, 2) == soar_gn.SOAR_EINVAL  # kernel size
    assert _dwf(L, 0, 8, 64, 64, 3, 2) == soar_gn.SOAR_OK  # empty


def test_pw_chunk_tuning(L):
    assert L.soar_gn_tune(soar_gn.TUNE_PW_CHUNK, 100) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_PW_CHUNK, 0) == soar_gn.SOAR_EINVAL
    soar_gn.tune(soar_gn.TUNE_PW_CHUNK, 2048)
    assert soar_gn.pw_conv_gn_workspace_bytes(1, 64, 2048 * 2048, 16) == (
        131072 * 16 + 1024 + 2 * 256 + 131072 * 8)
    soar_gn.tune(soar_gn.TUNE_PW_CHUNK, 1024)
    assert soar_gn.tune_get(soar_gn.TUNE_PW_CHUNK) == 1024


def test_pw_small_tuning(L):
    old = soar_gn.tune_get(soar_gn.TUNE_PW_SMALL)
    assert old == 1 << 25
    assert L.soar_gn_tune(soar_gn.TUNE_PW_SMALL, -1) == soar_gn.SOAR_EINVAL
    assert L.soar_gn_tune(soar_gn.TUNE_PW_SMALL, (1 << 40) + 1) == soar_gn.SOAR_EINVAL
    # small planes: the workspace also covers the GroupNorm's own plan
    big = soar_gn.pw_conv_gn_workspace_bytes(1, 512, 4, 8)
    soar_gn.tune(soar_gn.TUNE_PW_SMALL, 0)
    assert soar_gn.pw_conv_gn_workspace_bytes(1, 512, 4, 8) <= big
    soar_gn.tune(soar_gn.TUNE_PW_SMALL, old)
    assert soar_gn.tune_get(soar_gn.TUNE_PW_SMALL) == old


def test_pw_wg_waves_tuning(L):
    old = soar_gn.tune_get(soar_gn.TUNE_PW_WG_WAVES)
    assert old == 4
    for bad in (0, 3, 16, -1):
        assert L.soar_gn_tune(soar_gn.TUNE_PW_WG_WAVES, bad) == soar_gn.SOAR_EINVAL
    # the workspace holds one partial per chunk whatever the setting
    ws = soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 65536)
    for v in (1, 2, 8):
        soar_gn.tune(soar_gn.TUNE_PW_WG_WAVES, v)
        assert soar_gn.tune_get(soar_gn.TUNE_PW_WG_WAVES) == v
        assert soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 65536) == ws
    soar_gn.tune(soar_gn.TUNE_PW_WG_WAVES, old)


def test_pw_wg_target_tuning(L):
    old = soar_gn.tune_get(soar_gn.TUNE_PW_WG_TARGET)
    assert old == 2048
    for bad in (0, 255, (1 << 20) + 1):
        assert L.soar_gn_tune(soar_gn.TUNE_PW_WG_TARGET, bad) == soar_gn.SOAR_EINVAL
    # 65536 pixels, one tile: a target of 2048 waves gives chunks of 32
    # pixels, raised to the 64-pixel floor, so 1024 partial tiles.  A larger
    # target stays at the floor (same workspace); a smaller one gives longer
    # chunks and fewer partials.
    base = soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 65536)
    try:
        soar_gn.tune(soar_gn.TUNE_PW_WG_TARGET, 4096)
        assert soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 65536) == base
        soar_gn.tune(soar_gn.TUNE_PW_WG_TARGET, 512)
        assert soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 65536) < base
    finally:
        soar_gn.tune(soar_gn.TUNE_PW_WG_TARGET, old)


def test_fold_max_tuning(L):
    old = soar_gn.tune_get(soar_gn.TUNE_FOLD_MAX)
    assert old == 2048
    assert L.soar_gn_tune(soar_gn.TUNE_FOLD_MAX, 4097) == soar_gn.SOAR_EINVAL
    soar_gn.tune(soar_gn.TUNE_FOLD_MAX, 4096)
    assert soar_gn.tune_get(soar_gn.TUNE_FOLD_MAX) == 4096
    assert L.soar_gn_tune(soar_gn.TUNE_FOLD_MAX, -1) == soar_gn.SOAR_EINVAL
    soar_gn.tune(soar_gn.TUNE_FOLD_MAX, 0)
    assert soar_gn.tune_get(soar_gn.TUNE_FOLD_MAX) == 0
    soar_gn.tune(soar_gn.TUNE_FOLD_MAX, old)


def _cba(L, N, C_in, C_out, HW, G, flags=1, ws_bytes=0):
    """soar_pw_cba_backward with NULL tensors (validation runs first)."""
    P = [None] * 13
    P[9] = 1  # a non-NULL dx, so the call is not a no-op (never dereferenced)
    return L.soar_pw_cba_backward(*P, N, C_in, C_out, HW, G, flags, None, ws_bytes, None)


def test_pw_cba_backward_workspace_and_tuning(L):
    assert soar_gn.tune_get(soar_gn.TUNE_PW_CBA_MIN) == 1 << 14
    assert soar_gn.tune_get(soar_gn.TUNE_PW_CBA_BLOCKS) == 256
    gn = soar_gn.workspace_bytes(1, 64, 2048 * 2048, 16)
    # fused: the GroupNorm workspace (256-aligned), then 256 block partials
    # of the 64 x 64 weight gradient
    assert soar_gn.pw_cba_backward_workspace_bytes(1, 64, 64, 2048 * 2048, 16) == (
        (gn + 255) // 256 * 256 + 256 * 64 * 64 * 4)
    # below the size limit, or more than 64 channels: dz, the GroupNorm
    # workspace and the convolution backward's
    small = soar_gn.pw_cba_backward_workspace_bytes(1, 64, 64, 4096, 16)
    assert small >= 64 * 4096 * 4 + soar_gn.pw_conv_backward_workspace_bytes(1, 64, 64, 4096)
    # HW not a multiple of 4 as well
    assert soar_gn.pw_cba_backward_workspace_bytes(1, 64, 64, 65538, 16) >= 64 * 65538 * 4
    wide = soar_gn.pw_cba_backward_workspace_bytes(1, 64, 128, 1 << 18, 16)
    assert wide >= 128 * (1 << 18) * 4
    for bad in (-1, (1 << 40) + 1):
        assert L.soar_gn_tune(soar_gn.TUNE_PW_CBA_MIN, bad) == soar_gn.SOAR_EINVAL
    for bad in (63, (1 << 20) + 1):
        assert L.soar_gn_tune(soar_gn.TUNE_PW_CBA_BLOCKS, bad) == soar_gn.SOAR_EINVAL
    try:
        soar_gn.tune(soar_gn.TUNE_PW_CBA_BLOCKS, 1024)
        assert soar_gn.pw_cba_backward_workspace_bytes(1, 64, 64, 2048 * 2048, 16) == (
            (gn + 255) // 256 * 256 + 1024 * 64 * 64 * 4)
        soar_gn.tune(soar_gn.TUNE_PW_CBA_MIN, 0)  # never fused
        assert soar_gn.pw_cba_backward_workspace_bytes(1, 64, 64, 2048 * 2048, 16) > (
            64 * 2048 * 2048 * 4)
    finally:
        soar_gn.tune(soar_gn.TUNE_PW_CBA_BLOCKS, 256)
        soar_gn.tune(soar_gn.TUNE_PW_CBA_MIN, 1 << 14)
    assert soar_gn.pw_cba_backward_workspace_bytes(1, 64, 6, 4096, 4) == 0  # C_out % G
    assert soar_gn.pw_cba_backward_workspace_bytes(0, 64, 64, 4096, 4) == 0


def test_pw_cba_backward_validation_without_gpu(L):
    assert _cba(L, 1, 8, 6, 16, 4) == soar_gn.SOAR_EINVAL
    assert "divisible" in soar_gn.last_error()
    assert _cba(L, 1, 8, 6, 16, 3, flags=2) == soar_gn.SOAR_EINVAL  # no residual here
    assert "flags" in soar_gn.last_error()
    assert _cba(L, -1, 8, 6, 16, 3) == soar_gn.SOAR_EINVAL
    assert _cba(L, 1, 0, 6, 16, 3) == soar_gn.SOAR_EINVAL
    assert _cba(L, 1, 8, 6, 1 << 28, 3) == soar_gn.SOAR_EINVAL  # 32-bit offsets
    assert _cba(L, 0, 8, 6, 16, 3) == soar_gn.SOAR_OK  # empty
    assert _cba(L, 1, 8, 6, 0, 3) == soar_gn.SOAR_OK
    P = [None] * 13  # nothing requested
    assert L.soar_pw_cba_backward(*P, 1, 8, 6, 16, 3, 1, None, 0, None) == soar_gn.SOAR_OK


def _dwcba(L, N, C, H, W, Ho, Wo, K, pad, S, D, G, flags=1, ws_bytes=0, outputs=True):
    """soar_dw_cba_backward with NULL tensors (validation runs first)."""
    P = [None] * 13
    if outputs:
        P[9] = 1  # a non-NULL dx, so the call is not a no-op (never dereferenced)
    return L.soar_dw_cba_backward(*P, N, C, H, W, Ho, Wo, K, pad, S, D, G, flags, None,
                                  ws_bytes, None)


def test_dw_cba_backward_workspace_and_tuning(L):
    assert soar_gn.tune_get(soar_gn.TUNE_DW_CBA_MIN) == 1 << 14
    gn = (soar_gn.workspace_bytes(1, 64, 2048 * 2048, 16) + 255) // 256 * 256
    H = W = 2048
    # fused: the GroupNorm workspace, then one (K*K+1)-float partial per
    # channel and block; 32 x 64 tiles, 2 per block at k3, 64 at k7 (one
    # group per tile column of a 2048-row plane)
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H, W, 3, 1, 1, 1, 16) == (
        gn + 4 * (32 * 32) * 64 * 10)
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H, W, 7, 3, 1, 1, 16) == (
        gn + 4 * (1 * 32) * 64 * 50)
    dz = 64 * H * W * 4
    # outside the fused kernel (stride 2, padding other than "same", a K
    # without a tiled kernel): dz, the GroupNorm workspace, the conv backward's
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H // 2, W // 2, 3, 1, 2, 1,
                                                   16) >= dz // 4
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H - 2, W - 2, 3, 0, 1, 1,
                                                   16) >= 64 * (H - 2) * (W - 2) * 4
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H + 1, W + 1, 4, 2, 1, 1,
                                                   16) >= 64 * (H + 1) * (W + 1) * 4
    # below the size switch: unfused
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, 64, 64, 64, 64, 3, 1, 1, 1,
                                                   16) >= 64 * 64 * 64 * 4
    for bad in (-1, (1 << 40) + 1):
        assert L.soar_gn_tune(soar_gn.TUNE_DW_CBA_MIN, bad) == soar_gn.SOAR_EINVAL
    try:
        soar_gn.tune(soar_gn.TUNE_DW_CBA_MIN, 1)
        assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, 64, 64, 64, 64, 3, 1, 1, 1,
                                                       16) < 64 * 64 * 64 * 4
        soar_gn.tune(soar_gn.TUNE_DW_CBA_MIN, 0)  # never fused
        assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H, W, 3, 1, 1, 1, 16) > dz
    finally:
        soar_gn.tune(soar_gn.TUNE_DW_CBA_MIN, 1 << 14)
    assert soar_gn.dw_cba_backward_workspace_bytes(1, 64, H, W, H, W, 3, 1, 1, 1, 6) == 0
    assert soar_gn.dw_cba_backward_workspace_bytes(0, 64, H, W, H, W, 3, 1, 1, 1, 16) == 0


def test_dw_cba_backward_validation_without_gpu(L):
    args = (1, 8, 16, 16, 16, 16, 3, 1, 1, 1)
    assert _dwcba(L, *args, 3) == soar_gn.SOAR_EINVAL
    assert "divisible" in soar_gn.last_error()
    assert _dwcba(L, *args, 4, flags=2) == soar_gn.SOAR_EINVAL  # no residual here
    assert "flags" in soar_gn.last_error()
    assert _dwcba(L, -1, *args[1:], 4) == soar_gn.SOAR_EINVAL
    assert _dwcba(L, 1, 8, 16, 16, 16, 16, 0, 1, 1, 1, 4) == soar_gn.SOAR_EINVAL  # K = 0
    assert _dwcba(L, 1, 8, 16, 16, 16, 16, 3, 1, 0, 1, 4) == soar_gn.SOAR_EINVAL  # stride 0
    assert _dwcba(L, 0, *args[1:], 4) == soar_gn.SOAR_OK  # empty
    assert _dwcba(L, *args, 4, outputs=False) == soar_gn.SOAR_OK  # nothing requested
    assert _dwcba(L, *args, 4) == soar_gn.SOAR_ENODEV


def test_weight_finish_flag_and_flush_without_gpu(L):
    """SOAR_DEFER_WEIGHT_FINISH passes the convolution backward calls'
    validation (they then reach the device check); other flags bits and the
    GroupNorm calls still refuse it; with nothing queued the flush is a
    no-op on any stream."""
    D = soar_gn.DEFER_WEIGHT_FINISH
    assert L.soar_weight_grad_pending() == 0
    assert L.soar_weight_grad_flush(None) == soar_gn.SOAR_OK
    assert L.soar_weight_grad_flush(ctypes.c_void_p(0x1234)) == soar_gn.SOAR_OK
    nodev = L.soar_is_device_available() == 0
    rc = _cba(L, 1, 8, 6, 16, 3, flags=1 | D)
    assert rc == (soar_gn.SOAR_ENODEV if nodev else soar_gn.SOAR_EINVAL)
    assert _cba(L, 1, 8, 6, 16, 3, flags=1 | 16) == soar_gn.SOAR_EINVAL
    assert "flags" in soar_gn.last_error()
    args = (1, 8, 16, 16, 16, 16, 3, 1, 1, 1)
    if nodev:
        assert _dwcba(L, *args, 4, flags=1 | D) == soar_gn.SOAR_ENODEV
    assert _dwcba(L, *args, 4, flags=1 | 16) == soar_gn.SOAR_EINVAL
    dummy = ctypes.c_void_p(0x1000)
    P = [dummy, dummy, dummy, None, dummy, None]
    rc = L.soar_pw_conv_backward(*P, 1, 8, 6, 16, D, None, 0, None)
    if nodev:
        assert rc == soar_gn.SOAR_ENODEV
    assert L.soar_pw_conv_backward(*P, 1, 8, 6, 16, 16, None, 0, None) == soar_gn.SOAR_EINVAL
    rc = L.soar_dw_conv_backward(dummy, dummy, dummy, None, dummy, None, 1, 8, 16, 16, 16, 16, 3,
                                 1, 1, 1, D, None, 0, None)
    if nodev:
        assert rc == soar_gn.SOAR_ENODEV
    assert L.soar_dw_conv_backward(dummy, dummy, dummy, None, dummy, None, 1, 8, 16, 16, 16, 16,
                                   3, 1, 1, 1, 16, None, 0, None) == soar_gn.SOAR_EINVAL
    # the GroupNorm backward has no weight gradient to defer
    rc = L.soar_gn_silu_backward(None, None, None, None, None, None, None, None, None, None, 1, 6,
                                 16, 3, 1 | D, None, 0, None)
    assert rc == soar_gn.SOAR_EINVAL
    assert L.soar_weight_grad_pending() == 0
