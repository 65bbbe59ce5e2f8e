"""GPU parity of the fused entry points: PointwiseFuse chains (forward and the
y-style backward, directly and through teeny_dispatch), conv + BatchNorm +
activation (nn/fused/conv2d_bn_silu*.rs, all three dispatch variants with
their padded output rows), and whole graphs rewritten by the fusion passes
against the oracle and against the unfused graph."""
import ctypes

import numpy as np
import pytest

import teenygrad_amd as tg
from gpu_util import check_bf16, check_f32, check_f32_elementwise, stream_workspace
from teenygrad_amd import _lib, fusion
from teenygrad_amd import kernels as K
from teenygrad_amd.dtypes import from_bf16, round_bf16, to_bf16

pytestmark = pytest.mark.gpu


def up(dev, a, dtype):
    return dev.upload(to_bf16(a), tg.bf16) if dtype == "bf16" else dev.upload(np.ascontiguousarray(a, np.float32))


def host(buf, dtype):
    h = buf.to_host()
    return from_bf16(h).reshape(buf.shape) if dtype == "bf16" else h


CHAINS = [["relu", "sigmoid"], ["gelu", "silu", "tanh"], ["sigmoid", "tanh", "relu", "silu", "gelu"],
          ["tanh", "sigmoid", "relu"]]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("members", CHAINS)
@pytest.mark.parametrize("n", [4096 * 257, 10007])
def test_chain_forward(dev, orc, dtype, members, n):
    rng = np.random.default_rng(len(members) * 1000 + n % 97)
    x = rng.normal(0, 2.5, n).astype(np.float32)
    if dtype == "bf16":
        x = round_bf16(x)
    xb = up(dev, x, dtype)
    scratch = [tg.Buffer(xb.dtype, (n,)) for _ in members[:-1]]
    y = K.pointwise_chain(xb, members, scratch=scratch)
    ry, rs = orc.pointwise_chain(x, members, round_bf16 if dtype == "bf16" else None)
    print(f"[chain] {dtype} {members} n={n}", flush=True)
    if dtype == "f32":
        check_f32_elementwise(y.to_host(), ry, "y", rel=1e-5, floor=1e-6)
        for i, b in enumerate(scratch):
            check_f32_elementwise(b.to_host(), rs[i], f"scratch{i}", rel=1e-5, floor=1e-6)
    else:
        check_bf16(y.to_host(), ry, "y")
        for i, b in enumerate(scratch):
            check_bf16(b.to_host(), rs[i], f"scratch{i}")
    # without scratch (inference) the output is the same
    y2 = K.pointwise_chain(xb, members)
    np.testing.assert_array_equal(y2.to_host(), y.to_host())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_chain_equals_separate_kernels(dev, dtype):
    # the members exchange dtype-rounded values, as separate kernels do
    n = 1 << 20
    x = np.random.default_rng(3).normal(0, 2, n).astype(np.float32)
    xb = up(dev, x, dtype)
    seq = K.silu(K.gelu(K.relu(xb)))
    fused = K.pointwise_chain(xb, ["relu", "gelu", "silu"])
    np.testing.assert_array_equal(fused.to_host(), seq.to_host())


def test_chain_unaligned_and_in_place(dev, orc):
    n = 5003
    x = np.random.default_rng(4).normal(0, 2, n + 1).astype(np.float32)
    xb = dev.upload(x)
    ops = (ctypes.c_int32 * 2)(_lib.PW_SIGMOID, _lib.PW_TANH)
    yb = tg.Buffer(tg.f32, (n + 1,))
    tg.check(_lib.lib.teeny_pointwise_chain_forward(xb.ptr + 4, yb.ptr + 4, None, ops, 2, n, _lib.F32, None))
    check_f32_elementwise(yb.to_host()[1:], orc.pointwise_chain(x[1:], ["sigmoid", "tanh"])[0], "unaligned", rel=1e-5,
                          floor=1e-6)
    K.pointwise_chain(xb, ["sigmoid", "tanh"], y=xb)
    check_f32_elementwise(xb.to_host(), orc.pointwise_chain(x, ["sigmoid", "tanh"])[0], "in place", rel=1e-5,
                          floor=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("members", [["relu", "sigmoid"], ["tanh", "sigmoid", "relu"], ["sigmoid", "tanh"]])
def test_chain_backward(dev, orc, dtype, members):
    n = 300001
    rng = np.random.default_rng(11 + len(members))
    x = rng.normal(0, 2, n).astype(np.float32)
    dy = rng.normal(0, 1, n).astype(np.float32)
    rf = round_bf16 if dtype == "bf16" else None
    if dtype == "bf16":
        x, dy = round_bf16(x), round_bf16(dy)
    ry, rs = orc.pointwise_chain(x, members, rf)
    # the backward reads the forward's outputs: feed the oracle's, so both walk the same values
    yb = up(dev, ry, dtype)
    sb = [up(dev, s, dtype) for s in rs]
    dx = K.pointwise_chain_backward(up(dev, dy, dtype), yb, sb, members)
    rdx = orc.pointwise_chain_backward(dy, ry, rs, members, rf)
    if dtype == "f32":
        check_f32_elementwise(dx.to_host(), rdx, "dx", rel=1e-6, floor=1e-7)
    else:
        check_bf16(dx.to_host(), rdx, "dx")


def test_chain_backward_rejects_x_style_members(dev):
    b = tg.Buffer(tg.f32, (64,))
    with pytest.raises(tg.TeenyError) as e:
        K.pointwise_chain_backward(b, b, [b], ["gelu", "relu"])
    assert e.value.status == _lib.ERR_UNSUPPORTED


def test_pointwise_fuse_dispatch(dev, orc):
    # the PointwiseFuse RuntimeOp through teeny_dispatch, forward then backward
    n = 70000
    rng = np.random.default_rng(12)
    x = rng.normal(0, 2, n).astype(np.float32)
    dy = rng.normal(0, 1, n).astype(np.float32)
    op = K.PointwiseFuse(["relu", "sigmoid", "tanh"])
    xb, y = dev.upload(x), tg.Buffer(tg.f32, (n,))
    scratch = [tg.Buffer(tg.f32, (n,)) for _ in range(op.n_scratch)]
    op.launch([(xb, [n])], scratch, y, [n], tg.f32)
    ry, rs = orc.pointwise_chain(x, op.members)
    check_f32_elementwise(y.to_host(), ry, "y", rel=1e-5, floor=1e-6)
    dyb, dx = dev.upload(dy), tg.Buffer(tg.f32, (n,))
    packer = K.DispatchPacker()
    op.pack_backward_args([(xb, [n])], scratch, y, [n], dyb, n, [dx], [], packer)
    args, cnt = packer.array()
    grid = (ctypes.c_uint32 * 3)(*op.backward_grid([[n]], [n]))
    tg.check(_lib.lib.teeny_dispatch(op.backward_entry_point_name().encode(), (ctypes.c_int64 * 1)(0), 0, args, cnt,
                                     grid, _lib.F32, None))
    rdx = orc.pointwise_chain_backward(dy, y.to_host(), [s.to_host() for s in scratch], op.members)
    check_f32_elementwise(dx.to_host(), rdx, "dx", rel=1e-6, floor=1e-7)


# ── conv + BatchNorm + activation ───────────────────────────────────────────


def bn_params(rng, c):
    return rng.normal(1, 0.2, c).astype(np.float32), rng.normal(0, 0.3, c).astype(np.float32)


def oracle_conv_bn(orc, x, w, sc, sh, s, p, g, act):
    c = orc.conv2d_nchw(x, w, None, s, p, g)
    v = sc[None, :, None, None] * c + sh[None, :, None, None]
    return v if act is None else getattr(orc, act)(v)


@pytest.mark.parametrize("act", ["silu", "relu", "gelu", None])
@pytest.mark.parametrize("cfg", [(2, 16, 32, 14, 3, 1, 1, 1), (1, 8, 12, 9, 3, 2, 1, 4), (2, 64, 64, 8, 1, 1, 0, 1)])
def test_conv_bn_act_f32_nchw(dev, orc, act, cfg):
    B, cin, cout, H, k, s, p, g = cfg
    rng = np.random.default_rng(B * 31 + cin + cout + k)
    x = rng.normal(0, 1, (B, cin, H, H)).astype(np.float32)
    w = rng.normal(0, 0.2, (cout, cin // g, k, k)).astype(np.float32)
    sc, sh = bn_params(rng, cout)
    y = K.conv2d_bn_act(dev.upload(x), dev.upload(w), dev.upload(sc), dev.upload(sh), s, p, g, act).to_host()
    ref = orc.conv2d_bn_silu_nchw(x, w, sc, sh, s, p, g) if act == "silu" else oracle_conv_bn(orc, x, w, sc, sh, s, p,
                                                                                             g, act)
    check_f32(y, ref, f"conv+bn+{act}")


@pytest.mark.parametrize("act", ["silu", "relu", None])
@pytest.mark.parametrize("cfg", [(4, 64, 128, 14, 3, 1, 1), (2, 128, 256, 28, 1, 1, 0), (2, 3, 64, 32, 7, 2, 3),
                                 (2, 32, 48, 9, 3, 2, 1)])
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_conv_bn_act_bf16_nhwc(dev, orc, act, cfg, scratch):
    B, cin, cout, H, k, s, p = cfg
    rng = np.random.default_rng(B * 17 + cin + cout + k)
    x = round_bf16(rng.normal(0, 1, (B, H, H, cin)).astype(np.float32))
    w = round_bf16(rng.normal(0, 0.1, (cout, k, k, cin)).astype(np.float32))
    sc, sh = bn_params(rng, cout)
    xb, wb = dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16)
    need = K.conv2d_workspace_size(x.shape, w.shape, s, p, 1, tg.bf16, "nhwc")
    print(f"[conv bn bf16] {cfg} {act} {scratch} need={need}", flush=True)
    if scratch == "workspace":
        if need == 0:
            pytest.skip("no workspace plan for this shape")
        with stream_workspace(dev, need):
            y = K.conv2d_bn_act(xb, wb, dev.upload(sc), dev.upload(sh), s, p, 1, act, "nhwc")
            dev.synchronize()
    else:
        y = K.conv2d_bn_act(xb, wb, dev.upload(sc), dev.upload(sh), s, p, 1, act, "nhwc")
    ref = oracle_conv_bn(orc, x.transpose(0, 3, 1, 2), w.transpose(0, 3, 1, 2), sc, sh, s, p, 1, act)
    check_bf16(y.to_host(), np.ascontiguousarray(ref.transpose(0, 2, 3, 1)), f"conv+bn+{act}")


def test_conv_bn_silu_dispatch_variants(dev, orc):
    # the reference's three fused kernels through teeny_dispatch: plain, GEMM
    # (1x1, rows padded to BLOCK_M) and tiled (oh rows padded to BLOCK_OW); the
    # padding must stay untouched
    rng = np.random.default_rng(40)
    B, cin, cout, H = 2, 16, 24, 10
    x = rng.normal(0, 1, (B, cin, H, H)).astype(np.float32)
    sc, sh = bn_params(rng, cout)
    xb, scb, shb = dev.upload(x), dev.upload(sc), dev.upload(sh)
    # plain 3x3
    w3 = rng.normal(0, 0.2, (cout, cin, 3, 3)).astype(np.float32)
    op = K.Conv2dBnSiluForward(3, 3, 1, 1, 1, 1)
    y = tg.Buffer(tg.f32, (B, cout, H, H))
    op.launch([(xb, [B, cin, H, H])], [dev.upload(w3), scb, shb], y, [B, cout, H, H], tg.f32)
    check_f32(y.to_host(), orc.conv2d_bn_silu_nchw(x, w3, sc, sh, 1, 1), "plain")
    # GEMM 1x1: rows of OH*OW = 100 padded to 128
    w1 = rng.normal(0, 0.2, (cout, cin)).astype(np.float32)
    gop = K.Conv2dBnSiluGemmForward(128, 32, 32, 8)
    rs = gop.forward_output_row_stride([B, cout, H, H])
    assert rs == 128
    yg = dev.upload(np.full(B * cout * rs, 7.0, np.float32))
    gop.launch([(xb, [B, cin, H, H])], [dev.upload(w1), scb, shb], yg, [B, cout, H, H], tg.f32)
    got = yg.to_host().reshape(B, cout, rs)
    ref = orc.conv2d_bn_silu_nchw(x, w1.reshape(cout, cin, 1, 1), sc, sh)
    check_f32(got[:, :, :H * H].reshape(B, cout, H, H), ref, "gemm")
    assert np.all(got[:, :, H * H:] == 7.0)
    # tiled 3x3 stride 2: OW = 5 padded to 16 per oh row
    tp = K.Conv2dBnSiluTiledForward(3, 3, 2, 2, 1, 1, 16, 16)
    oh = 5
    cs = tp.forward_output_row_stride([B, cout, oh, oh])
    yt = dev.upload(np.full(B * cout * oh * cs, 7.0, np.float32))
    tp.launch([(xb, [B, cin, H, H])], [dev.upload(w3), scb, shb], yt, [B, cout, oh, oh], tg.f32)
    got = yt.to_host().reshape(B, cout, oh, cs)
    check_f32(got[..., :oh], orc.conv2d_bn_silu_nchw(x, w3, sc, sh, 2, 1), "tiled")
    assert np.all(got[..., oh:] == 7.0)


# ── graphs through the fusion passes ───────────────────────────────────────


def test_conv_bn_chain_graph(dev, orc):
    # conv -> batchnorm -> silu -> sigmoid -> tanh: conv2d_bn_act(silu) + a
    # [sigmoid, tanh] chain, against the oracle's unfused arithmetic
    rng = np.random.default_rng(50)
    B, cin, cout, H = 2, 8, 16, 12
    x = rng.normal(0, 1, (B, cin, H, H)).astype(np.float32)
    w = rng.normal(0, 0.2, (cout, cin, 3, 3)).astype(np.float32)
    gamma, beta = rng.normal(1, 0.1, cout), rng.normal(0, 0.1, cout)
    mean, var = rng.normal(0, 0.2, cout), rng.uniform(0.5, 1.5, cout)
    g = [fusion.Node("input", dtype="f32"),
         fusion.Node("conv2d", [0], {"weight": dev.upload(w), "padding": 1}, "f32"),
         fusion.Node("batchnorm", [1], {"gamma": gamma, "beta": beta, "mean": mean, "var": var}, "f32"),
         fusion.Node("silu", [2], dtype="f32"), fusion.Node("sigmoid", [3], dtype="f32"),
         fusion.Node("tanh", [4], dtype="f32")]
    fused = fusion.optimize(g)
    assert [n.op for n in fused] == ["input", "conv2d_bn_act", "pointwise_fuse"]
    out = fusion.run(fused, {0: dev.upload(x)}, dev)
    sc, sh = K.fold_batchnorm(gamma, beta, mean, var)
    ref = orc.conv2d_bn_silu_nchw(x, w, sc, sh, 1, 1)
    ref = orc.pointwise_chain(ref, ["sigmoid", "tanh"])[0]
    check_f32(out[-1].to_host(), ref, "graph")


@pytest.mark.parametrize("rms", [False, True])
def test_norm_chain_graph_vs_unfused(dev, orc, rms):
    # norm -> gelu -> relu -> sigmoid (bf16): the fused graph (norm_act + chain)
    # against the same graph run op by op
    rng = np.random.default_rng(60 + rms)
    m, n = 512, 1024
    x = round_bf16(rng.normal(0, 1, (m, n)).astype(np.float32))
    wt = round_bf16(rng.normal(1, 0.1, n).astype(np.float32))
    bs = round_bf16(rng.normal(0, 0.1, n).astype(np.float32))
    attrs = {"weight": up(dev, wt, "bf16")} if rms else {"weight": up(dev, wt, "bf16"), "bias": up(dev, bs, "bf16")}
    g = [fusion.Node("input"), fusion.Node("rms_norm" if rms else "layer_norm", [0], attrs), fusion.Node("gelu", [1]),
         fusion.Node("relu", [2]), fusion.Node("sigmoid", [3])]
    fused = fusion.optimize(g)
    assert [n.op for n in fused] == ["input", "rms_norm" if rms else "layer_norm", "pointwise_fuse"]
    assert fused[1].attrs["act"] == "gelu" and fused[2].attrs["members"] == ["relu", "sigmoid"]
    xb = up(dev, x, "bf16")
    a = fusion.run(fused, {0: xb}, dev)[-1].to_host()
    b = fusion.run(g, {0: xb}, dev)[-1].to_host()
    # the unfused graph rounds the norm output to bf16 before the GELU
    check_bf16(a, from_bf16(b), "fused vs unfused")
    nrm = orc.rms_norm(x, wt, 1e-8)[0] if rms else orc.layer_norm(x, wt, bs, 1e-5)
    ref = orc.pointwise_chain(orc.gelu(nrm), ["relu", "sigmoid"], round_bf16)[0]
    check_bf16(a, ref, "fused vs oracle")
