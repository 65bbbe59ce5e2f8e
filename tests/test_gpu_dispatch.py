"""GPU: the reference-shaped dispatch path.  Each op is driven the way the
reference executor drives it — RuntimeOp.pack_args + RuntimeOp.grid, then the
"{name}_entry_point" launch (drivers/teeny-cuda/src/model/mod.rs:524-700) —
through teeny_dispatch, and checked against the reference fixtures."""
import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from teenygrad_amd import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cls,op,tol", [(K.ReluForward, "relu", 0.0), (K.GeluForward, "gelu", 2e-5),
                                        (K.SiluForward, "silu", 1e-5)])
def test_elementwise(dev, cls, op, tol):
    x = load_golden(f"{op}/x.bin")
    xb, yb = dev.upload(x), tg.Buffer(tg.f32, x.shape)
    cls(1024).launch([(xb, x.shape)], [], yb, list(x.shape), tg.f32)
    assert np.max(np.abs(yb.to_host() - load_golden(f"{op}/expected_forward.bin"))) <= tol


def test_layernorm(dev):
    x = load_golden("layernorm/x.bin").reshape(16, 128)
    op = K.LayerNormForwardInferenceRuntimeOp(1024, 1e-5)
    y = tg.Buffer(tg.f32, (16, 128))
    op.launch([(dev.upload(x), [16, 128])],
              [dev.upload(load_golden("layernorm/weight.bin")), dev.upload(load_golden("layernorm/bias.bin"))],
              y, [16, 128], tg.f32)
    assert np.max(np.abs(y.to_host() - load_golden("layernorm/expected_forward.bin").reshape(16, 128))) < 1e-4


def test_rmsnorm(dev):
    x = load_golden("rmsnorm/x.bin").reshape(16, 128)
    op = K.RmsNormForwardRuntimeOp(1024, 1e-8)
    y, rr = tg.Buffer(tg.f32, (16, 128)), tg.Buffer(tg.f32, (16,))
    op.launch([(dev.upload(x), [16, 128])], [dev.upload(load_golden("rmsnorm/weight.bin")), rr], y,
              [16, 128], tg.f32)
    assert np.max(np.abs(y.to_host() - load_golden("rmsnorm/expected_forward.bin").reshape(16, 128))) < 1e-4
    assert np.max(np.abs(rr.to_host() - load_golden("rmsnorm/expected_rrms.bin"))) < 1e-4


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_conv2d(dev, orc, case, pad, oh):
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    y = tg.Buffer(tg.f32, (1, 4, oh, oh))
    K.Conv2dForward(3, 3, 1, 1, pad, pad, 1, 8).launch([(dev.upload(x), [1, 2, 8, 8])], [dev.upload(w)], y,
                                                        [1, 4, oh, oh], tg.f32)
    want = load_golden(f"{case}/expected_forward.bin").reshape(1, 4, oh, oh)
    assert np.max(np.abs(y.to_host() - want)) < 1e-4
    # the fused-bias kernel (conv2d.rs:642-764) with a bias vector
    b = np.array([0.5, -0.25, 0.125, 1.0], np.float32)
    yb = tg.Buffer(tg.f32, (1, 4, oh, oh))
    K.Conv2dBiasForward(3, 3, 1, 1, pad, pad, 1, 16).launch([(dev.upload(x), [1, 2, 8, 8])],
                                                             [dev.upload(w), dev.upload(b)], yb,
                                                             [1, 4, oh, oh], tg.f32)
    assert np.max(np.abs(yb.to_host() - (want + b[None, :, None, None]))) < 1e-4


def test_flash_attention(dev):
    shape = [4, 8, 64]
    q, k, v = (dev.upload(load_golden(f"flash_attn2/{n}.bin").reshape(shape)) for n in "qkv")
    o, l = tg.Buffer(tg.f32, shape), tg.Buffer(tg.f32, (4, 8))
    K.FlashAttention2Forward(64, 0.125).launch([(q, shape), (k, shape), (v, shape)], [l], o, shape, tg.f32)
    assert np.max(np.abs(o.to_host() - load_golden("flash_attn2/expected_forward_o.bin").reshape(shape))) < 1e-4
    assert np.max(np.abs(l.to_host() - load_golden("flash_attn2/expected_forward_l.bin").reshape(4, 8))) < 1e-4


@pytest.mark.parametrize("use_bias", [False, True])
def test_linear(dev, use_bias):
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    b = load_golden("linear/bias.bin")
    y = tg.Buffer(tg.f32, (64, 48))
    params = [dev.upload(w)] + ([dev.upload(b)] if use_bias else [])
    K.LinearForward(use_bias).launch([(dev.upload(x), [64, 64])], params, y, [64, 48], tg.f32)
    want = load_golden(f"linear/expected_{'with' if use_bias else 'no'}_bias.bin").reshape(64, 48)
    np.testing.assert_allclose(y.to_host(), want, rtol=0.02, atol=0.1)


@pytest.mark.parametrize("cls,op,tol", [(K.ReluForward, "relu", 0.0), (K.GeluForward, "gelu", 2e-5),
                                        (K.SiluForward, "silu", 1e-5)])
def test_elementwise_backward(dev, cls, op, tol):
    # RuntimeOp.pack_backward_args + backward_grid through "<op>_backward_entry_point"
    # (relu.rs:148-180, gelu.rs:287-317, sigmoid.rs:418-448), against the reference's
    # backward fixtures (test_relu.rs:148, test_gelu.rs:157, test_sigmoid.rs:274)
    import ctypes
    from teenygrad_amd._lib import check, lib
    if op == "relu":
        saved, dy = load_golden("relu/y_backward.bin"), load_golden("relu/dy_backward.bin")
    else:
        saved, dy = load_golden(f"{op}/x.bin"), load_golden(f"{op}/dy.bin")
    shape = list(saved.shape)
    sb, dyb, dxb = dev.upload(saved), dev.upload(dy), tg.Buffer(tg.f32, saved.shape)
    rop = cls(1024)
    packer = K.DispatchPacker()
    # forward output (relu) or forward input (gelu/silu) as the saved tensor
    rop.pack_backward_args([(sb, shape)], [], sb, shape, dyb, shape[-1], [dxb], [], packer)
    args, n = packer.array()
    cg = (ctypes.c_int64 * 1)(*rop.const_generics())
    grid = (ctypes.c_uint32 * 3)(*rop.backward_grid([shape], shape))
    check(lib.teeny_dispatch(rop.backward_entry_point_name().encode(), cg, 1, args, n, grid, tg.f32.code, None))
    assert np.max(np.abs(dxb.to_host() - load_golden(f"{op}/expected_backward.bin"))) <= tol


def _rb(a):
    from teenygrad_amd.dtypes import from_bf16, to_bf16
    return from_bf16(to_bf16(a))


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_causal_const_generic(dev, orc, causal):
    # flash_attention2_forward<HEAD_DIM, CAUSAL>: the optional CAUSAL const generic
    from gpu_util import check_bf16
    from teenygrad_amd.dtypes import to_bf16
    rng = np.random.default_rng(21)
    shape = [3, 150, 128]
    q, k, v = (_rb(rng.standard_normal(shape, dtype=np.float32)) for _ in range(3))
    qb, kb, vb = (dev.upload(to_bf16(t), tg.bf16) for t in (q, k, v))
    o, l = tg.Buffer(tg.bf16, shape), tg.Buffer(tg.f32, (3, 150))
    op = K.FlashAttention2Forward(128, None, causal)
    assert op.const_generics() == ((128, 1) if causal else (128,))
    op.launch([(qb, shape), (kb, shape), (vb, shape)], [l], o, shape, tg.bf16)
    oo, ol = orc.flash_attention(q, k, v, causal=causal)
    check_bf16(o.to_host(), oo, "o")
    assert np.max(np.abs(l.to_host() - ol)) < 1e-3


@pytest.mark.parametrize("hq,hkv,causal,dt", [(8, 2, True, "bf16"), (4, 4, False, "bf16"), (6, 3, True, "f32"),
                                              (4, 1, False, "f32")])
def test_multi_head_attention(dev, orc, hq, hkv, causal, dt):
    # Op::MultiHeadAttention{q_num_heads, kv_num_heads} lowered onto the flash kernel:
    # grouped K/V heads equal ordinary attention on K/V heads repeated per group
    from gpu_util import check_bf16, check_f32
    from teenygrad_amd.dtypes import to_bf16
    B, nq, nk, d = 2, 130, 97, 64
    rng = np.random.default_rng(hq * 10 + hkv)
    q = _rb(rng.standard_normal((B * hq, nq, d), dtype=np.float32))
    k = _rb(rng.standard_normal((B * hkv, nk, d), dtype=np.float32))
    v = _rb(rng.standard_normal((B * hkv, nk, d), dtype=np.float32))
    up = (lambda a: dev.upload(to_bf16(a), tg.bf16)) if dt == "bf16" else dev.upload
    dtype = tg.bf16 if dt == "bf16" else tg.f32
    o, l = tg.Buffer(dtype, (B * hq, nq, d)), tg.Buffer(tg.f32, (B * hq, nq))
    op = K.MultiHeadAttentionRuntimeOp(hq, hkv, d, causal)
    assert op.grid([B * hq, nq, d]) == (nq, B * hq, 1)
    op.launch([(up(q), list(q.shape)), (up(k), list(k.shape)), (up(v), list(v.shape))], [l], o,
              [B * hq, nq, d], dtype)
    g = hq // hkv
    kr = np.repeat(k.reshape(B, hkv, nk, d), g, axis=1).reshape(B * hq, nk, d)
    vr = np.repeat(v.reshape(B, hkv, nk, d), g, axis=1).reshape(B * hq, nk, d)
    oo, ol = orc.flash_attention(q, kr, vr, causal=causal)
    if dt == "bf16":
        check_bf16(o.to_host(), oo, "mha o")
        assert np.max(np.abs(l.to_host() - ol)) < 1e-3
    else:
        check_f32(o.to_host(), oo, "mha o")
        check_f32(l.to_host(), ol, "mha l")


@pytest.mark.parametrize("use_bias,act", [(False, None), (True, "silu")])
def test_w8a16_linear_dispatch(dev, orc, use_bias, act):
    from gpu_util import check_bf16
    from teenygrad_amd.dtypes import to_bf16
    m, n, k = 200, 320, 256
    rng = np.random.default_rng(5)
    x = _rb(rng.standard_normal((m, k), dtype=np.float32))
    wf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, s, _, _ = orc.quantize_affine(wf, [n, k], "channel", 0)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    y = tg.Buffer(tg.bf16, (m, n))
    params = [dev.upload(q.reshape(n, k)), dev.upload(s)] + ([dev.upload(bias)] if use_bias else [])
    K.W8A16LinearRuntimeOp(use_bias, act).launch([(dev.upload(to_bf16(x), tg.bf16), [m, k])], params, y,
                                                 [m, n], tg.bf16)
    ref = orc.w8a16_linear(x, q.reshape(n, k), s, bias if use_bias else None)
    if act:
        ref = orc.silu(ref)
    check_bf16(y.to_host(), ref, "w8a16 dispatch")


def test_w8a16_conv_dispatch(dev, orc):
    from gpu_util import check_bf16
    from teenygrad_amd.dtypes import to_bf16
    B, H, cin, cout = 2, 14, 64, 96
    rng = np.random.default_rng(6)
    x = _rb(rng.standard_normal((B, H, H, cin), dtype=np.float32))
    wf = rng.normal(0, 0.02, (cout, 3, 3, cin)).astype(np.float32)
    q, s, _, _ = orc.quantize_affine(wf, list(wf.shape), "channel", 0)
    bias = rng.normal(0, 0.1, cout).astype(np.float32)
    y = tg.Buffer(tg.bf16, (B, 7, 7, cout))
    op = K.W8A16Conv2dRuntimeOp(3, 3, 2, 2, 1, 1, 1, 16, True, "relu")
    op.launch([(dev.upload(to_bf16(x), tg.bf16), [B, H, H, cin])],
              [dev.upload(q.reshape(wf.shape)), dev.upload(s), dev.upload(bias)], y, [B, 7, 7, cout], tg.bf16)
    wdeq = orc.dequantize_affine(q, s, None, list(wf.shape), "channel", 0)
    ref = orc.relu(orc.conv2d_nhwc(x, wdeq, bias, stride=2, padding=1))
    check_bf16(y.to_host(), ref, "w8a16 conv dispatch")


@pytest.mark.parametrize("gran,axis,gs,sym", [("channel", 0, 1, True), ("group", 1, 8, False), ("tensor", 0, 1, True)])
def test_quantize_dequantize_dispatch(dev, orc, gran, axis, gs, sym):
    shape = [12, 40]
    x = np.random.default_rng(7).normal(0, 0.05, shape).astype(np.float32)
    ng = K.quant_num_groups(shape, gran, axis, gs)
    qb, sb, zb = tg.Buffer(tg.i8, shape), tg.Buffer(tg.f32, (ng,)), tg.Buffer("i32", (ng,))
    K.QuantizeAffineRuntimeOp(gran, axis, gs, sym, 8).launch([(dev.upload(x), shape)], [sb, zb], qb, shape, tg.f32)
    oq, os_, oz, _ = orc.quantize_affine(x, shape, gran, axis, gs, sym, 8)
    np.testing.assert_array_equal(qb.to_host().reshape(-1), oq)
    np.testing.assert_array_equal(sb.to_host(), os_)
    np.testing.assert_array_equal(zb.to_host(), oz)
    out = tg.Buffer(tg.f32, shape)
    K.DequantizeAffineRuntimeOp(gran, axis, gs).launch([(qb, shape)], [sb, zb], out, shape, tg.f32)
    np.testing.assert_array_equal(out.to_host(), orc.dequantize_affine(oq, os_, oz, shape, gran, axis, gs))


# ── training kernels through teeny_dispatch ────────────────────────────────


def _dispatch(name, cgs, fill, grid, dtype=tg.f32):
    import ctypes
    from teenygrad_amd._lib import check, lib
    packer = K.DispatchPacker()
    fill(packer)
    args, n = packer.array()
    cg = (ctypes.c_int64 * max(1, len(cgs)))(*cgs)
    g = (ctypes.c_uint32 * 3)(*grid)
    check(lib.teeny_dispatch(name.encode(), cg, len(cgs), args, n, g, dtype.code, None))


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_conv2d_backward_hooks(dev, case, pad, oh):
    # Conv2dForward's pack_backward_args + backward_grid through
    # "conv2d_backward_entry_point" (conv2d.rs:574-617), against test_conv2d.rs's
    # backward fixtures; then the separate dx / dw kernels (conv2d.rs:172-311)
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    dy = load_golden(f"{case}/dy.bin").reshape(1, 4, oh, oh)
    want_dx = load_golden(f"{case}/expected_dx.bin").reshape(x.shape)
    want_dw = load_golden(f"{case}/expected_dw.bin").reshape(w.shape)
    xb, wb, dyb = dev.upload(x), dev.upload(w), dev.upload(dy)
    dx, dw = tg.Buffer(tg.f32, x.shape), tg.Buffer(tg.f32, w.shape)
    op = K.Conv2dForward(3, 3, 1, 1, pad, pad)
    yshape = [1, 4, oh, oh]
    _dispatch(op.backward_entry_point_name(), op.const_generics(),
              lambda p: op.pack_backward_args([(xb, list(x.shape))], [wb], None, yshape, dyb, oh, [dx], [dw], p),
              op.backward_grid([list(x.shape)], yshape))
    assert np.max(np.abs(dx.to_host() - want_dx)) < 1e-4
    assert np.max(np.abs(dw.to_host() - want_dw)) < 1e-3
    dx2, dw2 = tg.Buffer(tg.f32, x.shape), tg.Buffer(tg.f32, w.shape)
    dims = (1, 2, 4, 8, 8, oh, oh)

    def fill_dx(p):
        for b in (dyb, wb, dx2):
            p.visit_ptr(b)
        for d in dims:
            p.visit_i32(d)

    def fill_dw(p):
        for b in (dyb, xb, dw2):
            p.visit_ptr(b)
        for d in dims:
            p.visit_i32(d)

    _dispatch("conv2d_backward_dx_entry_point", op.const_generics(), fill_dx, op.grid(yshape))
    _dispatch("conv2d_backward_dw_entry_point", op.const_generics(), fill_dw, op.grid(yshape))
    np.testing.assert_array_equal(dx2.to_host(), dx.to_host())
    np.testing.assert_array_equal(dw2.to_host(), dw.to_host())


def test_layer_norm_training_dispatch(dev, orc):
    # layer_norm_forward (layernorm.rs:163-172) and layer_norm_backward (:301-311)
    # on the reference's layernorm fixture inputs
    from gpu_util import check_f32
    x = load_golden("layernorm/x.bin")
    w, b = load_golden("layernorm/weight.bin"), load_golden("layernorm/bias.bin")
    n = w.size
    m = x.size // n
    dy = np.random.default_rng(5).normal(0, 1, x.size).astype(np.float32)
    xb, wb, bb, dyb = (dev.upload(a) for a in (x, w, b, dy))
    y, mean, rstd = tg.Buffer(tg.f32, (x.size,)), tg.Buffer(tg.f32, (m,)), tg.Buffer(tg.f32, (m,))

    def fill_fwd(p):
        for t in (xb, y, wb, bb, mean, rstd):
            p.visit_ptr(t)
        p.visit_i32(m)
        p.visit_i32(n)
        p.visit_f32(1e-5)

    _dispatch("layer_norm_forward_entry_point", (1024,), fill_fwd, (m, 1, 1))
    np.testing.assert_allclose(y.to_host(), load_golden("layernorm/expected_forward.bin"), atol=1e-4)
    ry, rmean, rrstd = orc.layer_norm_train(x.reshape(m, n), w, b, 1e-5)
    check_f32(mean.to_host(), rmean, "mean")
    check_f32(rstd.to_host(), rrstd, "rstd")
    dx, dwt, dbt = tg.Buffer(tg.f32, (x.size,)), dev.upload(np.zeros(n, np.float32)), dev.upload(
        np.zeros(n, np.float32))

    def fill_bwd(p):
        for t in (dyb, xb, dx, wb, dwt, dbt, mean, rstd):
            p.visit_ptr(t)
        p.visit_i32(m)
        p.visit_i32(n)

    _dispatch("layer_norm_backward_entry_point", (1024,), fill_bwd, (m, 1, 1))
    rdx, rdw, rdb = orc.layer_norm_backward(dy.reshape(m, n), x.reshape(m, n), w, rmean, rrstd)
    check_f32(dx.to_host(), rdx, "dx")
    check_f32(dwt.to_host(), rdw, "dweight")
    check_f32(dbt.to_host(), rdb, "dbias")


def test_rms_norm_backward_dispatch(dev, orc):
    # rms_norm_backward (rmsnorm.rs:136-144) from the fixture's rrms
    from gpu_util import check_f32
    x, w = load_golden("rmsnorm/x.bin"), load_golden("rmsnorm/weight.bin")
    rrms = load_golden("rmsnorm/expected_rrms.bin")
    n, m = w.size, rrms.size
    dy = np.random.default_rng(6).normal(0, 1, x.size).astype(np.float32)
    xb, wb, rb_, dyb = (dev.upload(a) for a in (x, w, rrms, dy))
    dx, dwt = tg.Buffer(tg.f32, (x.size,)), dev.upload(np.zeros(n, np.float32))

    def fill(p):
        for t in (dyb, xb, dx, wb, dwt, rb_):
            p.visit_ptr(t)
        p.visit_i32(m)
        p.visit_i32(n)

    _dispatch("rms_norm_backward_entry_point", (1024,), fill, (m, 1, 1))
    rdx, rdw = orc.rms_norm_backward(dy.reshape(m, n), x.reshape(m, n), w, rrms)
    check_f32(dx.to_host(), rdx, "dx")
    check_f32(dwt.to_host(), rdw, "dweight")


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_backward_dispatch(dev, orc, causal):
    # flash_attention2_backward_dq / _dkv (flash_attn2.rs:174-185, :312-324) with the
    # reference grids (n_ctx_q, BH, 1) / (n_ctx_k, BH, 1); the reference fixture
    # (non-causal) and the oracle
    from gpu_util import check_f32
    shape = (4, 8, 64)
    q, k, v, do = (load_golden(f"flash_attn2/{n}.bin").reshape(shape) for n in ("q", "k", "v", "do"))
    o, l = orc.flash_attention(q, k, v, 0.125, causal)
    bufs = [dev.upload(a) for a in (q, k, v, o, do, l)]
    dq, dk, dv = (tg.Buffer(tg.f32, shape) for _ in range(3))
    cgs = (64, 1) if causal else (64,)

    def fill(outs):
        def f(p):
            for t in bufs + outs:
                p.visit_ptr(t)
            p.visit_i32(8)
            p.visit_i32(8)
            p.visit_f32(0.125)
        return f

    _dispatch("flash_attention2_backward_dq_entry_point", cgs, fill([dq]), (8, 4, 1))
    _dispatch("flash_attention2_backward_dkv_entry_point", cgs, fill([dk, dv]), (8, 4, 1))
    rq, rk, rv = orc.flash_attention_backward(q, k, v, o, do, l, 0.125, causal)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        g = got.to_host()
        check_f32(g, ref, name)
        if not causal:
            assert np.max(np.abs(g - load_golden(f"flash_attn2/expected_backward_{name}.bin").reshape(shape))) < 1e-3
