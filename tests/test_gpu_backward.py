"""GPU parity of the training kernels: LayerNorm / RMSNorm forward statistics
and backward, conv2d dx / dw, against the reference fixtures
(tests/golden/conv2d*, the backward checks of test_conv2d.rs) and the CPU
oracle's restatement of layernorm.rs:162-482, rmsnorm.rs:135-277 and
conv2d.rs:171-397 on the same seeded inputs."""
import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from gpu_util import check_bf16, check_bf16_normwise, check_f32, stream_workspace
from teenygrad_amd import kernels as K
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def rb(a):
    return from_bf16(to_bf16(a)).reshape(a.shape)


def up(dev, a, dtype):
    return dev.upload(to_bf16(a), tg.bf16) if dtype == "bf16" else dev.upload(np.ascontiguousarray(a, np.float32))


def check(dtype, got_buf, ref, what):
    got = got_buf.to_host()
    return check_bf16(got, ref, what) if dtype == "bf16" else check_f32(got, ref, what)


# ── LayerNorm / RMSNorm ─────────────────────────────────────────────────────

NORM_CASES = [  # (M, N): register plans VPT 1/2/4, ragged N, the multipass kernel; 773 rows
    # give the row kernel's workgroups (one per CU) three or four rows each, so its three-row
    # unrolled loop leaves at each of its exits
    (300, 1024), (257, 2048), (64, 4096), (33, 8192), (50, 1000), (17, 12288), (7, 77), (773, 512)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,n", NORM_CASES)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_layer_norm_backward(dev, orc, dtype, m, n, scratch):
    rng = np.random.default_rng(m * 7919 + n)
    x = rng.normal(0.5, 2, (m, n)).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    dy = rng.normal(0, 1, (m, n)).astype(np.float32)
    if dtype == "bf16":
        x, w, b, dy = rb(x), rb(w), rb(b), rb(dy)
    dw0 = rng.normal(0, 1, n).astype(np.float32)
    db0 = rng.normal(0, 1, n).astype(np.float32)
    print(f"[ln bwd] {dtype} M={m} N={n} {scratch}", flush=True)
    xb, wb, bb, dyb = up(dev, x, dtype), up(dev, w, dtype), up(dev, b, dtype), up(dev, dy, dtype)
    # training forward: y plus the statistics
    y, mean, rstd = K.layer_norm_train(xb, wb, bb, 1e-5)
    ry, rmean, rrstd = orc.layer_norm_train(x, w, b, 1e-5)
    check(dtype, y, ry, "layer_norm_train y")
    check_f32(mean.to_host(), rmean, "mean")
    check_f32(rstd.to_host(), rrstd, "rstd")
    # backward from the oracle's statistics
    dwb, dbb = dev.upload(dw0), dev.upload(db0)
    need = K.norm_backward_workspace_size(m, n, False, tg.bf16 if dtype == "bf16" else tg.f32)
    args = (dyb, xb, wb, dev.upload(rmean), dev.upload(rrstd), dwb, dbb)
    if scratch == "workspace":
        if need == 0:
            pytest.skip("no workspace plan for this shape")
        with stream_workspace(dev, need):
            dx = K.layer_norm_backward(*args)
            dev.synchronize()
    else:
        dx = K.layer_norm_backward(*args)
    rdx, rdw, rdb = orc.layer_norm_backward(dy, x, w, rmean, rrstd, dw0, db0)
    check(dtype, dx, rdx, "layer_norm_backward dx")
    check_f32(dwb.to_host(), rdw, "dweight")
    check_f32(dbb.to_host(), rdb, "dbias")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,n", NORM_CASES)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_rms_norm_backward(dev, orc, dtype, m, n, scratch):
    rng = np.random.default_rng(m * 104729 + n)
    x = rng.normal(0.3, 1.5, (m, n)).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    dy = rng.normal(0, 1, (m, n)).astype(np.float32)
    if dtype == "bf16":
        x, w, dy = rb(x), rb(w), rb(dy)
    dw0 = rng.normal(0, 1, n).astype(np.float32)
    print(f"[rms bwd] {dtype} M={m} N={n} {scratch}", flush=True)
    xb, wb, dyb = up(dev, x, dtype), up(dev, w, dtype), up(dev, dy, dtype)
    _, rrms = orc.rms_norm(x, w, 1e-8)
    dwb = dev.upload(dw0)
    need = K.norm_backward_workspace_size(m, n, True, tg.bf16 if dtype == "bf16" else tg.f32)
    args = (dyb, xb, wb, dev.upload(rrms), dwb)
    if scratch == "workspace":
        if need == 0:
            pytest.skip("no workspace plan for this shape")
        with stream_workspace(dev, need):
            dx = K.rms_norm_backward(*args)
            dev.synchronize()
    else:
        dx = K.rms_norm_backward(*args)
    rdx, rdw = orc.rms_norm_backward(dy, x, w, rrms, dw0)
    check(dtype, dx, rdx, "rms_norm_backward dx")
    check_f32(dwb.to_host(), rdw, "dweight")


def test_norm_backward_skips_param_grads(dev, orc):
    # dweight / dbias NULL: dx only
    rng = np.random.default_rng(11)
    m, n = 40, 512
    x, dy = rng.normal(0, 1, (m, n)).astype(np.float32), rng.normal(0, 1, (m, n)).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    _, mean, rstd = orc.layer_norm_train(x, w, np.zeros(n, np.float32))
    dx = K.layer_norm_backward(dev.upload(dy), dev.upload(x), dev.upload(w), dev.upload(mean), dev.upload(rstd))
    check_f32(dx.to_host(), orc.layer_norm_backward(dy, x, w, mean, rstd)[0], "dx only")


@pytest.mark.parametrize("which", ["dweight", "dbias"])
def test_layer_norm_backward_one_param_grad(dev, orc, which):
    # with the workspace, only one of dweight / dbias requested: the column
    # sums run for that one alone
    rng = np.random.default_rng(23 if which == "dweight" else 29)
    m, n = 300, 1024
    x, dy = rng.normal(0, 1, (m, n)).astype(np.float32), rng.normal(0, 1, (m, n)).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    _, mean, rstd = orc.layer_norm_train(x, w, np.zeros(n, np.float32))
    g0 = rng.normal(0, 1, n).astype(np.float32)
    gb = dev.upload(g0)
    need = K.norm_backward_workspace_size(m, n, False, tg.f32)
    print(f"[ln bwd one grad] {which} workspace {need} B", flush=True)
    kw = {which: gb}
    with stream_workspace(dev, need):
        dx = K.layer_norm_backward(dev.upload(dy), dev.upload(x), dev.upload(w), dev.upload(mean), dev.upload(rstd),
                                   **kw)
        dev.synchronize()
    rdx, rdw, rdb = orc.layer_norm_backward(dy, x, w, mean, rstd, g0, g0)
    check_f32(dx.to_host(), rdx, "dx")
    check_f32(gb.to_host(), rdw if which == "dweight" else rdb, which)


def test_layer_norm_backward_config(dev, orc):
    # the norm workload's shape: X[16384, 4096] bf16, with the stream workspace
    m, n = 16384, 4096
    rng = np.random.default_rng(0x7EE70002)
    x = rb(rng.standard_normal((m, n), dtype=np.float32))
    dy = rb(rng.standard_normal((m, n), dtype=np.float32))
    w = rb(rng.normal(1, 0.2, n).astype(np.float32))
    b = rb(rng.normal(0, 0.1, n).astype(np.float32))
    print(f"[ln bwd] bf16 [{m}, {n}] config", flush=True)
    xb, dyb, wb, bb = (dev.upload(to_bf16(a), tg.bf16) for a in (x, dy, w, b))
    _, mean, rstd = K.layer_norm_train(xb, wb, bb, 1e-5)
    _, rmean, rrstd = orc.layer_norm_train(x, w, b, 1e-5)
    check_f32(mean.to_host(), rmean, "mean")
    check_f32(rstd.to_host(), rrstd, "rstd")
    dwb, dbb = dev.upload(np.zeros(n, np.float32)), dev.upload(np.zeros(n, np.float32))
    with stream_workspace(dev, K.norm_backward_workspace_size(m, n, False)):
        dx = K.layer_norm_backward(dyb, xb, wb, mean, rstd, dwb, dbb)
        dev.synchronize()
    rdx, rdw, rdb = orc.layer_norm_backward(dy, x, w, rmean, rrstd)
    check_bf16(dx.to_host(), rdx, "dx")
    check_f32(dwb.to_host(), rdw, "dweight")
    check_f32(dbb.to_host(), rdb, "dbias")


# ── conv2d dx / dw ───────────────────────────────────────────────────────────


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_conv_backward_fixtures(dev, orc, case, pad, oh):
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    dy = load_golden(f"{case}/dy.bin").reshape(1, 4, oh, oh)
    dyb, xb, wb = dev.upload(dy), dev.upload(x), dev.upload(w)
    dx = K.conv2d_backward_dx(dyb, wb, x.shape, 1, pad).to_host()
    dw = K.conv2d_backward_dw(dyb, xb, w.shape, 1, pad).to_host()
    # the reference test's bounds, then the oracle
    assert np.max(np.abs(dx - load_golden(f"{case}/expected_dx.bin").reshape(x.shape))) < 1e-4
    assert np.max(np.abs(dw - load_golden(f"{case}/expected_dw.bin").reshape(w.shape))) < 1e-3
    check_f32(dx, orc.conv2d_backward_dx(dy, w, x.shape, 1, pad), "dx")
    check_f32(dw, orc.conv2d_backward_dw(dy, x, w.shape, 1, pad), "dw")


CONV_CASES = [  # B, Cin, Cout, H, W, K, stride, pad, groups
    (2, 3, 5, 9, 11, 3, 1, 1, 1),
    (2, 4, 6, 10, 10, 3, 2, 1, 2),
    (1, 6, 4, 13, 7, (3, 1), (2, 1), (1, 0), 1),
    (3, 8, 8, 8, 8, 1, 2, 0, 4),
    (2, 3, 8, 15, 15, 7, 2, 3, 1),
    (1, 4, 4, 6, 6, 5, 3, 2, 1),
]


def nhwc_of(a):
    return np.ascontiguousarray(a.transpose(0, 2, 3, 1))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
@pytest.mark.parametrize("cfg", CONV_CASES)
def test_conv_backward_direct(dev, orc, dtype, layout, cfg):
    B, cin, cout, H, W, k, s, p, g = cfg
    kh, kw = (k, k) if isinstance(k, int) else k
    rng = np.random.default_rng(abs(hash(cfg)) % 2 ** 32)
    x = rng.normal(0, 1, (B, cin, H, W)).astype(np.float32)
    w = rng.normal(0, 0.3, (cout, cin // g, kh, kw)).astype(np.float32)
    sh, sw = (s, s) if isinstance(s, int) else s
    ph, pw = (p, p) if isinstance(p, int) else p
    oh, ow = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    dy = rng.normal(0, 1, (B, cout, oh, ow)).astype(np.float32)
    if dtype == "bf16":
        x, w, dy = rb(x), rb(w), rb(dy)
    print(f"[conv bwd] {dtype} {layout} {cfg}", flush=True)
    rdx = orc.conv2d_backward_dx(dy, w, x.shape, (sh, sw), (ph, pw), g)
    rdw = orc.conv2d_backward_dw(dy, x, w.shape, (sh, sw), (ph, pw), g)
    if layout == "nhwc":
        xs, ws_, dys = nhwc_of(x), nhwc_of(w), nhwc_of(dy)
        rdx, rdw = nhwc_of(rdx), nhwc_of(rdw)
    else:
        xs, ws_, dys = x, w, dy
    dyb, xb, wb = up(dev, dys, dtype), up(dev, xs, dtype), up(dev, ws_, dtype)
    dx = K.conv2d_backward_dx(dyb, wb, xs.shape, (sh, sw), (ph, pw), g, layout)
    dw = K.conv2d_backward_dw(dyb, xb, ws_.shape, (sh, sw), (ph, pw), g, layout)
    check(dtype, dx, rdx, "dx")
    check(dtype, dw, rdw, "dw")


MFMA_DX_CASES = [  # bf16 NHWC, groups 1: B, H, Cin, Cout, K, stride, pad (ResNet-50 shapes)
    (4, 14, 64, 128, 3, 1, 1),
    (4, 28, 128, 128, 3, 2, 1),
    (4, 28, 256, 512, 1, 2, 0),
    (2, 56, 64, 256, 1, 1, 0),
    (2, 30, 3, 64, 7, 2, 3),
    (3, 9, 32, 64, 3, 2, 0),
    # strided convs run as their sub-pixel phases (one stride-1 GEMM per
    # (ih % S, iw % S) class, remapped output rows; phases without taps zeroed)
    (4, 28, 256, 256, 3, 2, 1),   # the ResNet-50 stage-3 downsampling 3x3
    # 3x3/2 pad 1 with 14- or 28-wide dy: the four phases in one band-tiled
    # launch (units of phase, image band and 64 input channels)
    (3, 56, 128, 128, 3, 2, 1),   # the stage-2 downsampling 3x3 (28-wide dy)
    (2, 56, 64, 64, 3, 2, 1),
    (40, 28, 192, 64, 3, 2, 1),   # 480 units: several per workgroup, channel tiles changing
    (2, 15, 64, 64, 3, 2, 1),     # odd H: phases of 8 and 7 rows
    (2, 13, 32, 48, 5, 3, 2),     # stride 3, 5x5
    (2, 12, 16, 32, 4, 2, 1),     # even kernel
    (2, 30, 16, 64, 7, 2, 3),     # stem-like 7x7/2: 4 x 4, 4 x 3, 3 x 4, 3 x 3 taps
    (3, 14, 64, 128, 1, 2, 0),    # 1x1/2 on even H: odd rows and columns are zero
]


@pytest.mark.parametrize("cfg", MFMA_DX_CASES)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_conv_backward_dx_bf16_nhwc(dev, orc, cfg, scratch):
    B, H, cin, cout, k, s, p = cfg
    rng = np.random.default_rng(B * 1000 + H * 10 + cin + cout)
    oh = (H + 2 * p - k) // s + 1
    x_shape = (B, H, H, cin)
    w = rb(rng.normal(0, 0.1, (cout, k, k, cin)).astype(np.float32))
    dy = rb(rng.normal(0, 1, (B, oh, oh, cout)).astype(np.float32))
    need = K.conv2d_backward_workspace_size(x_shape, w.shape, s, p, 1, tg.bf16, "nhwc")
    print(f"[conv dx mfma] {cfg} {scratch} need={need}", flush=True)
    if scratch == "workspace" and need == 0:
        pytest.skip("no MFMA plan for this shape")
    dyb, wb = dev.upload(to_bf16(dy), tg.bf16), dev.upload(to_bf16(w), tg.bf16)
    if scratch == "workspace":
        with stream_workspace(dev, need):
            dx = K.conv2d_backward_dx(dyb, wb, x_shape, s, p, 1, "nhwc")
            dev.synchronize()
    else:
        dx = K.conv2d_backward_dx(dyb, wb, x_shape, s, p, 1, "nhwc")
    ref = orc.conv2d_backward_dx(dy.transpose(0, 3, 1, 2), w.transpose(0, 3, 1, 2), (B, cin, H, H), s, p)
    check_bf16(dx.to_host(), nhwc_of(ref), "dx")


MFMA_DW_CASES = [  # bf16 NHWC, groups 1: B, H, Cin, Cout, K, stride, pad
    (4, 14, 64, 128, 3, 1, 1),
    (2, 28, 128, 128, 3, 2, 1),
    (3, 7, 512, 256, 1, 1, 0),
    (2, 15, 24, 72, 3, 1, 1),     # ragged: N = 216, C_OUT = 72, pixels 450
    (1, 11, 40, 200, 5, 2, 2),    # 5x5 stride 2, N = 1000
    (2, 30, 8, 64, 7, 2, 3),
    # few tiles over many pixels: with a workspace the pixel range splits 20
    # and 10 ways (the split sum loads eight partials at a time, then a tail)
    (8, 28, 64, 64, 3, 1, 1),
    (16, 14, 32, 32, 3, 1, 1),
]


@pytest.mark.parametrize("cfg", MFMA_DW_CASES)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_conv_backward_dw_bf16_nhwc(dev, orc, cfg, scratch):
    B, H, cin, cout, k, s, p = cfg
    rng = np.random.default_rng(B * 7 + H * 100 + cin + 3 * cout)
    oh = (H + 2 * p - k) // s + 1
    x = rb(rng.normal(0, 1, (B, H, H, cin)).astype(np.float32))
    dy = rb(rng.normal(0, 1, (B, oh, oh, cout)).astype(np.float32))
    w_shape = (cout, k, k, cin)
    need = K.conv2d_backward_workspace_size(x.shape, w_shape, s, p, 1, tg.bf16, "nhwc")
    print(f"[conv dw mfma] {cfg} {scratch} need={need}", flush=True)
    dyb, xb = dev.upload(to_bf16(dy), tg.bf16), dev.upload(to_bf16(x), tg.bf16)
    if scratch == "workspace":
        with stream_workspace(dev, need):
            dw = K.conv2d_backward_dw(dyb, xb, w_shape, s, p, 1, "nhwc")
            dev.synchronize()
    else:
        dw = K.conv2d_backward_dw(dyb, xb, w_shape, s, p, 1, "nhwc")
    ref = nhwc_of(orc.conv2d_backward_dw(dy.transpose(0, 3, 1, 2), x.transpose(0, 3, 1, 2), (cout, cin, k, k), s, p))
    got = dw.to_host()
    check_bf16(got, ref, "dw")
    print(f"  dw norm-wise {check_bf16_normwise(got, ref, 'dw'):.3g}", flush=True)


def test_conv_backward_combined_and_dispatch_hooks(dev, orc):
    # teeny_conv2d_backward (dx and dw in one call) and the Conv2dForward
    # RuntimeOp's backward hooks (conv2d.rs:574-617)
    rng = np.random.default_rng(21)
    B, cin, cout, H = 2, 4, 8, 10
    x = rng.normal(0, 1, (B, cin, H, H)).astype(np.float32)
    w = rng.normal(0, 0.3, (cout, cin, 3, 3)).astype(np.float32)
    dy = rng.normal(0, 1, (B, cout, H, H)).astype(np.float32)
    dyb, xb, wb = dev.upload(dy), dev.upload(x), dev.upload(w)
    dx, dw = tg.Buffer(tg.f32, x.shape), tg.Buffer(tg.f32, w.shape)
    import ctypes
    from teenygrad_amd import _lib
    prm = _lib.Conv2dParams(3, 3, 1, 1, 1, 1, 1, 0)
    tg.check(_lib.lib.teeny_conv2d_backward(dyb.ptr, xb.ptr, wb.ptr, dx.ptr, dw.ptr, B, cin, cout, H, H, H, H,
                                            ctypes.byref(prm), _lib.F32, _lib.NCHW, None))
    check_f32(dx.to_host(), orc.conv2d_backward_dx(dy, w, x.shape, 1, 1), "dx")
    check_f32(dw.to_host(), orc.conv2d_backward_dw(dy, x, w.shape, 1, 1), "dw")
    op = K.Conv2dForward(3, 3, 1, 1, 1, 1)
    assert op.has_backward()


def test_conv_backward_empty_batch_zeroes_dw(dev):
    # no images: dw is the sum over no pixels, written as zeros
    w_shape = (8, 4, 3, 3)
    dw = dev.upload(np.full(w_shape, 5.0, np.float32))
    dy, x = tg.Buffer(tg.f32, (1, 8, 6, 6)), tg.Buffer(tg.f32, (1, 4, 6, 6))
    import ctypes
    from teenygrad_amd import _lib
    prm = _lib.Conv2dParams(3, 3, 1, 1, 1, 1, 1, 0)
    tg.check(_lib.lib.teeny_conv2d_backward_dw(dy.ptr, x.ptr, dw.ptr, 0, 4, 8, 6, 6, 6, 6, ctypes.byref(prm),
                                               _lib.F32, _lib.NCHW, None))
    np.testing.assert_array_equal(dw.to_host(), 0.0)


# ── linear backward ─────────────────────────────────────────────────────────
# linear_backward, kernels/teeny-kernels/src/nn/mlp/linear.rs:118-250:
# dx = dy W, dw = dy^T x, db = column sums of dy.


def test_linear_backward_fixture(dev):
    # test_linear.rs:434-626: M=64, N=48, K=64 fp32, with and without bias
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    dy = load_golden("linear/dy.bin").reshape(64, 48)
    for use_bias in (True, False):
        print(f"[linear bwd fixture] bias={use_bias}", flush=True)
        dx, dw, db = K.linear_backward(dev.upload(x), dev.upload(w), dev.upload(dy), use_bias)
        check_f32(dx.to_host(), load_golden("linear/expected_dx.bin"), "dx")
        check_f32(dw.to_host(), load_golden("linear/expected_dw.bin"), "dw")
        if use_bias:
            check_f32(db.to_host(), load_golden("linear/expected_db.bin"), "db")
        else:
            assert db is None


LINEAR_BWD = [  # (M, N, K): the matrix-core plan (N, K multiples of 8) and the generic kernel
    (512, 256, 384), (4096, 1024, 512), (100, 40, 24), (37, 30, 20), (3, 8, 8)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m,n,k", LINEAR_BWD)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_linear_backward(dev, orc, dtype, m, n, k, scratch):
    rng = np.random.default_rng(m + 7 * n + 13 * k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.1))
    dy = rb(rng.standard_normal((m, n), dtype=np.float32))
    tdt = tg.bf16 if dtype == "bf16" else tg.f32
    need = K.linear_backward_workspace_size(m, n, k, tdt)
    if scratch == "workspace" and need == 0:
        pytest.skip("no workspace plan at this shape")
    print(f"[linear bwd] {dtype} M={m} N={n} K={k} workspace={need if scratch == 'workspace' else 0}", flush=True)
    xb, wb, dyb = up(dev, x, dtype), up(dev, w, dtype), up(dev, dy, dtype)

    def run():
        return K.linear_backward(xb, wb, dyb)

    if scratch == "workspace":
        with stream_workspace(dev, need):
            dx, dw, db = run()
    else:
        dx, dw, db = run()
    rdx, rdw, rdb = orc.linear_backward(x, w, dy)
    check(dtype, dx, rdx, "dx")
    check(dtype, dw, rdw, "dw")
    check(dtype, db, rdb, "db")
    if dtype == "bf16":  # gradients near zero next to the 2e-2 bound: also norm-wise
        check_bf16_normwise(dw.to_host(), rdw, "dw")


def test_linear_backward_strided_and_empty(dev, orc):
    # x given transposed in memory (stride_xm 1, stride_xk M) and dy rows
    # padded to 16 bytes (the RuntimeOp's backward_grad_output_row_stride):
    # the generic kernel reads any strides
    import ctypes
    from teenygrad_amd._lib import check as chk, lib
    rng = np.random.default_rng(11)
    m, n, k, pad = 50, 21, 33, 24
    x = rng.standard_normal((m, k), dtype=np.float32)
    w = rng.standard_normal((n, k), dtype=np.float32)
    dy = rng.standard_normal((m, n), dtype=np.float32)
    dyp = np.zeros((m, pad), np.float32)
    dyp[:, :n] = dy
    # every device buffer stays referenced until the call has completed
    xt, wb, dyb = dev.upload(np.ascontiguousarray(x.T)), dev.upload(w), dev.upload(dyp)
    dx, dw, db = tg.Buffer(tg.f32, (m, k)), tg.Buffer(tg.f32, (n, k)), tg.Buffer(tg.f32, (n,))
    chk(lib.teeny_linear_backward(xt.ptr, wb.ptr, dyb.ptr, dx.ptr, dw.ptr, db.ptr, m, n, k,
                                  1, m, 1, k, pad, 1, k, 1, 1, k, 1, tg.f32.code, None))
    rdx, rdw, rdb = orc.linear_backward(x, w, dy)
    check_f32(dx.to_host(), rdx, "dx strided")
    check_f32(dw.to_host(), rdw, "dw strided")
    check_f32(db.to_host(), rdb, "db strided")
    # M = 0: no rows, so dw and db are sums over nothing (zero); dx is empty
    dw0, db0 = dev.upload(np.full((n, k), 7.0, np.float32)), dev.upload(np.full(n, 7.0, np.float32))
    chk(lib.teeny_linear_backward(None, wb.ptr, None, None, dw0.ptr, db0.ptr, 0, n, k, k, 1, 1, k, n, 1,
                                  k, 1, 1, k, 1, tg.f32.code, None))
    assert not np.any(dw0.to_host()) and not np.any(db0.to_host())


@pytest.mark.parametrize("use_bias", [True, False])
def test_linear_backward_runtime_op(dev, use_bias):
    # LinearForward.pack_backward_args + backward_grid through
    # "linear_backward_entry_point" (linear.rs:322-385), against the fixtures
    import ctypes
    from teenygrad_amd._lib import check as chk, lib
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    dy = load_golden("linear/dy.bin").reshape(64, 48)
    op = K.LinearForward(use_bias, 32, 32, 32, 8)
    xb, wb, dyb = dev.upload(x), dev.upload(w), dev.upload(dy)
    dx, dw = tg.Buffer(tg.f32, (64, 64)), tg.Buffer(tg.f32, (48, 64))
    db = tg.Buffer(tg.f32, (48,))
    packer = K.DispatchPacker()
    op.pack_backward_args([(xb, [64, 64])], [wb], None, [64, 48], dyb, op.backward_grad_output_row_stride([64, 48]), [dx],
                          [dw] + ([db] if use_bias else []), packer)
    args, n = packer.array()
    cg = (ctypes.c_int64 * 5)(*op.const_generics())
    grid = (ctypes.c_uint32 * 3)(*op.backward_grid([[64, 64]], [64, 48]))
    assert tuple(grid) == (2 * 2 * 2, 1, 1)
    chk(lib.teeny_dispatch(op.backward_entry_point_name().encode(), cg, 5, args, n, grid, tg.f32.code, None))
    check_f32(dx.to_host(), load_golden("linear/expected_dx.bin"), "dx")
    check_f32(dw.to_host(), load_golden("linear/expected_dw.bin"), "dw")
    if use_bias:
        check_f32(db.to_host(), load_golden("linear/expected_db.bin"), "db")
