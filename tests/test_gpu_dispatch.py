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
