"""The oracle's fused-op restatements, pinned without a GPU: sigmoid / tanh
(sigmoid.rs, tanh.rs) against float64 closed forms and torch autograd, the
PointwiseFuse chain (graph/optimizer/ops/pointwise_fuse.rs) against its
members run one at a time, and conv2d_bn_silu (nn/fused/conv2d_bn_silu.rs)
against conv2d + affine + SiLU and torch."""
import numpy as np
import pytest
import torch

RNG = np.random.default_rng(0x7EE7F0)


def rel_inf(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def test_sigmoid_tanh_closed_forms(orc):
    x = np.concatenate([np.linspace(-30, 30, 4001), RNG.normal(0, 3, 2000)]).astype(np.float32)
    x64 = x.astype(np.float64)
    s = orc.sigmoid(x)
    t = orc.tanh(x)
    assert np.max(np.abs(s - 1 / (1 + np.exp(-x64)))) < 2e-7
    assert np.max(np.abs(t - np.tanh(x64))) < 4e-7
    # special values: saturation and the zero crossing
    assert orc.sigmoid(np.array([0.0, 100.0, -100.0], np.float32)).tolist() == [0.5, 1.0, 0.0]
    assert orc.tanh(np.array([0.0, 50.0, -50.0], np.float32)).tolist() == [0.0, 1.0, -1.0]


@pytest.mark.parametrize("name", ["sigmoid", "tanh", "relu"])
def test_y_style_gradients_vs_autograd(orc, name):
    x = RNG.normal(0, 2, 3000).astype(np.float32)
    dy = RNG.normal(0, 1, 3000).astype(np.float32)
    y = getattr(orc, name)(x)
    dx = getattr(orc, name + "_backward")(dy, y)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    getattr(torch, name)(xt).backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dx, xt.grad.numpy()) < 2e-6


@pytest.mark.parametrize("members", [["relu", "sigmoid"], ["gelu", "silu", "tanh"],
                                     ["sigmoid", "tanh", "relu", "silu", "gelu"]])
def test_chain_is_members_in_order(orc, members):
    x = RNG.normal(0, 2, 5000).astype(np.float32)
    y, scratch = orc.pointwise_chain(x, members)
    v = x
    for i, m in enumerate(members):
        v = getattr(orc, m)(v)
        if i + 1 < len(members):
            np.testing.assert_array_equal(scratch[i], v)
    np.testing.assert_array_equal(y, v)
    # and the composition against float64 torch
    t = torch.tensor(x, dtype=torch.float64)
    f = {"relu": torch.relu, "sigmoid": torch.sigmoid, "tanh": torch.tanh, "silu": torch.nn.functional.silu,
         "gelu": lambda a: torch.nn.functional.gelu(a, approximate="tanh")}
    for m in members:
        t = f[m](t)
    assert rel_inf(y, t.numpy()) < 1e-5


@pytest.mark.parametrize("members", [["relu", "sigmoid"], ["tanh", "sigmoid", "relu"], ["sigmoid", "tanh"]])
def test_chain_backward_vs_autograd(orc, members):
    x = RNG.normal(0, 2, 4000).astype(np.float32)
    dy = RNG.normal(0, 1, 4000).astype(np.float32)
    y, scratch = orc.pointwise_chain(x, members)
    dx = orc.pointwise_chain_backward(dy, y, scratch, members)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    t = xt
    for m in members:
        t = getattr(torch, m)(t)
    t.backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dx, xt.grad.numpy()) < 1e-5


def test_chain_sensitivity(orc):
    # a dropped member or a swapped order must show
    x = RNG.normal(0, 2, 1000).astype(np.float32)
    y, _ = orc.pointwise_chain(x, ["sigmoid", "tanh"])
    assert rel_inf(orc.pointwise_chain(x, ["tanh", "sigmoid"])[0], y) > 1e-2
    assert rel_inf(orc.tanh(x), y) > 1e-2


@pytest.mark.parametrize("cfg", [(2, 6, 4, 9, 11, 3, (2, 1), (1, 1), 2), (1, 3, 8, 7, 7, 1, 1, 0, 1),
                                 (2, 4, 4, 10, 10, 5, 2, 2, 4)])
def test_conv_bn_silu(orc, cfg):
    B, cin, cout, H, W, k, s, p, g = cfg
    x = RNG.normal(0, 1, (B, cin, H, W)).astype(np.float32)
    w = RNG.normal(0, 0.3, (cout, cin // g, k, k)).astype(np.float32)
    sc = RNG.normal(1, 0.2, cout).astype(np.float32)
    sh = RNG.normal(0, 0.3, cout).astype(np.float32)
    y = orc.conv2d_bn_silu_nchw(x, w, sc, sh, s, p, g)
    c = orc.conv2d_nchw(x, w, None, s, p, g)
    # the reference's epilogue order: scale * acc + shift, then SiLU
    np.testing.assert_array_equal(y, orc.silu(sc[None, :, None, None] * c + sh[None, :, None, None]))
    ss = (s, s) if isinstance(s, int) else s
    t = torch.nn.functional.conv2d(torch.tensor(x, dtype=torch.float64), torch.tensor(w, dtype=torch.float64),
                                   stride=ss, padding=p, groups=g)
    t = t * torch.tensor(sc, dtype=torch.float64)[None, :, None, None] + torch.tensor(sh, dtype=torch.float64)[
        None, :, None, None]
    assert rel_inf(y, torch.nn.functional.silu(t).numpy()) < 1e-5


def test_fold_batchnorm_matches_batchnorm():
    from teenygrad_amd.kernels import fold_batchnorm
    c = 16
    gamma, beta = RNG.normal(1, 0.2, c), RNG.normal(0, 0.2, c)
    mean, var = RNG.normal(0, 0.5, c), RNG.uniform(0.5, 2.0, c)
    x = RNG.normal(0, 1, (4, c, 5, 5))
    scale, shift = fold_batchnorm(gamma, beta, mean, var, 1e-5)
    bn = torch.nn.functional.batch_norm(torch.tensor(x), torch.tensor(mean), torch.tensor(var), torch.tensor(gamma),
                                        torch.tensor(beta), training=False, eps=1e-5).numpy()
    assert rel_inf(x * scale[None, :, None, None] + shift[None, :, None, None], bn) < 1e-6
