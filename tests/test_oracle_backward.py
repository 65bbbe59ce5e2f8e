"""Pinning the oracle's backward restatements (CPU only).

conv2d dx/dw and flash-attention dq/dk/dv against the reference's own
fixtures (tests/golden/*/expected_d*.bin, the tolerances of the reference's
tests), and every backward function against float64 torch autograd on the CPU
(an independent differentiation of the forward formulas) and, for the norms,
against central finite differences of a float64 restatement of the forward.
Sensitivity checks show that a dropped term or a transposed operand fails."""
import numpy as np
import pytest
import torch

from conftest import load_golden

RNG = np.random.default_rng(2026)


def rel_inf(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ── conv2d: the reference fixtures (test_conv2d.rs backward checks) ──────────


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_conv_backward_fixtures(orc, case, pad, oh):
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    dy = load_golden(f"{case}/dy.bin").reshape(1, 4, oh, oh)
    dx = orc.conv2d_backward_dx(dy, w, x.shape, 1, pad)
    dw = orc.conv2d_backward_dw(dy, x, w.shape, 1, pad)
    assert np.max(np.abs(dx - load_golden(f"{case}/expected_dx.bin").reshape(x.shape))) < 1e-4
    assert np.max(np.abs(dw - load_golden(f"{case}/expected_dw.bin").reshape(w.shape))) < 1e-3


CONV_CASES = [  # B, Cin, Cout, H, W, KH, KW, stride, pad, groups
    (2, 3, 5, 9, 7, 3, 3, (1, 1), (1, 1), 1), (1, 4, 6, 11, 10, 3, 2, (2, 3), (1, 0), 2),
    (1, 6, 6, 8, 8, 3, 3, (1, 1), (1, 1), 6), (2, 8, 4, 7, 7, 1, 1, (2, 2), (0, 0), 1),
    (1, 3, 4, 16, 15, 7, 7, (2, 2), (3, 3), 1), (2, 4, 8, 10, 10, 3, 3, (2, 2), (1, 1), 1),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_backward_vs_torch_autograd(orc, case):
    B, Cin, Cout, H, W, KH, KW, st, pd, G = case
    x = RNG.normal(0, 1, (B, Cin, H, W)).astype(np.float32)
    w = RNG.normal(0, 0.3, (Cout, Cin // G, KH, KW)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.conv2d(xt, wt, stride=st, padding=pd, groups=G)
    dy = RNG.normal(0, 1, tuple(y.shape)).astype(np.float32)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    dx = orc.conv2d_backward_dx(dy, w, x.shape, st, pd, G)
    dw = orc.conv2d_backward_dw(dy, x, w.shape, st, pd, G)
    assert rel_inf(dx, xt.grad.numpy()) < 1e-5
    assert rel_inf(dw, wt.grad.numpy()) < 1e-5


def test_conv_backward_sensitivity(orc):
    # the flipped-kernel (convolution instead of correlation) gradient must fail
    x = RNG.normal(0, 1, (1, 2, 8, 8)).astype(np.float32)
    w = RNG.normal(0, 0.3, (3, 2, 3, 3)).astype(np.float32)
    dy = RNG.normal(0, 1, (1, 3, 8, 8)).astype(np.float32)
    dx = orc.conv2d_backward_dx(dy, w, x.shape, 1, 1)
    wrong = orc.conv2d_backward_dx(dy, w[:, :, ::-1, ::-1].copy(), x.shape, 1, 1)
    assert rel_inf(wrong, dx) > 1e-2


# ── flash attention backward: the reference fixture (test_flash_attn2.rs) ───


def test_flash_attention_backward_fixture(orc):
    shape = (4, 8, 64)
    q, k, v, do = (load_golden(f"flash_attn2/{n}.bin").reshape(shape) for n in ("q", "k", "v", "do"))
    o, l = orc.flash_attention(q, k, v, 0.125)
    dq, dk, dv = orc.flash_attention_backward(q, k, v, o, do, l, 0.125)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        want = load_golden(f"flash_attn2/expected_backward_{name}.bin").reshape(shape)
        assert np.max(np.abs(got - want)) < 1e-3, name


@pytest.mark.parametrize("bh,nq,nk,d,causal", [(2, 17, 17, 32, False), (2, 17, 17, 32, True), (1, 9, 23, 64, True),
                                               (3, 20, 12, 16, False)])
def test_flash_attention_backward_vs_torch(orc, bh, nq, nk, d, causal):
    q = RNG.normal(0, 1, (bh, nq, d)).astype(np.float32)
    k = RNG.normal(0, 1, (bh, nk, d)).astype(np.float32)
    v = RNG.normal(0, 1, (bh, nk, d)).astype(np.float32)
    do = RNG.normal(0, 1, (bh, nq, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    qt, kt, vt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    s = (qt @ kt.transpose(1, 2)) * scale
    if causal:
        s = s.masked_fill(torch.ones(nq, nk, dtype=torch.bool).triu(1), float("-inf"))
    (torch.softmax(s, -1) @ vt).backward(torch.tensor(do, dtype=torch.float64))
    o, l = orc.flash_attention(q, k, v, scale, causal)
    dq, dk, dv = orc.flash_attention_backward(q, k, v, o, do, l, scale, causal)
    assert rel_inf(dq, qt.grad.numpy()) < 1e-4
    assert rel_inf(dk, kt.grad.numpy()) < 1e-4
    assert rel_inf(dv, vt.grad.numpy()) < 1e-4


def test_flash_attention_backward_sensitivity(orc):
    # a causal gradient taken with the non-causal oracle must fail
    q, k, v, do = (RNG.normal(0, 1, (1, 12, 16)).astype(np.float32) for _ in range(4))
    o, l = orc.flash_attention(q, k, v, None, True)
    dq, dk, dv = orc.flash_attention_backward(q, k, v, o, do, l, None, True)
    dq2, dk2, dv2 = orc.flash_attention_backward(q, k, v, o, do, l, None, False)
    assert rel_inf(dv2, dv) > 1e-2 and rel_inf(dk2, dk) > 1e-2


# ── LayerNorm / RMSNorm backward ───────────────────────────────────────────
# The reference's formulas (the doc comments of layernorm.rs:284-297 and
# rmsnorm.rs:126-133) apply gamma outside the bracket:
#   LN:  dx = rstd * g * (dy - mean(dy g) - xhat * mean(dy g xhat))
#   RMS: dx = rrms * g * (dy - x rrms^2 * mean(dy g x))
# which is the true gradient of the forward when g == 1 (torch autograd and
# finite differences pin that case) and the reference's own closed form
# otherwise (evaluated here in float64 from the doc comment).  dweight and
# dbias are the true gradients for every g.


def ln64(x, w, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def rms64(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def ln_ref_formula64(dy, x, w, eps):
    x, dy, w = (a.astype(np.float64) for a in (x, dy, w))
    mu = x.mean(-1, keepdims=True)
    rstd = 1.0 / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
    xhat = (x - mu) * rstd
    return rstd * w * (dy - (dy * w).mean(-1, keepdims=True) - xhat * (dy * w * xhat).mean(-1, keepdims=True))


def rms_ref_formula64(dy, x, w, eps):
    x, dy, w = (a.astype(np.float64) for a in (x, dy, w))
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return r * w * (dy - x * r * r * (dy * w * x).mean(-1, keepdims=True))


@pytest.mark.parametrize("m,n,block", [(5, 128, 1024), (3, 1000, 256), (4, 37, 16)])
def test_layernorm_backward(orc, m, n, block):
    x = RNG.normal(0.5, 2, (m, n)).astype(np.float32)
    b = RNG.normal(0, 0.1, n).astype(np.float32)
    dy = RNG.normal(0, 1, (m, n)).astype(np.float32)
    dw0 = RNG.normal(0, 1, n).astype(np.float32)  # dweight/dbias accumulate into what is there
    # gamma == 1: the true gradient (torch autograd, finite differences)
    w1 = np.ones(n, np.float32)
    y, mean, rstd = orc.layer_norm_train(x, w1, b, 1e-5, block)
    assert rel_inf(y, orc.layer_norm(x, w1, b, 1e-5, block)) == 0.0  # same arithmetic as inference
    dx, dw, db = orc.layer_norm_backward(dy, x, w1, mean, rstd, dw0, dw0, block)
    xt, wt, bt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w1, b))
    torch.nn.functional.layer_norm(xt, (n,), wt, bt, 1e-5).backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dx, xt.grad.numpy()) < 1e-4
    assert rel_inf(dw - dw0, wt.grad.numpy()) < 1e-4
    assert rel_inf(db - dw0, bt.grad.numpy()) < 1e-5
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    u = RNG.normal(0, 1, (m, n))
    h = 1e-6
    fd = ((ln64(x64 + h * u, w1, b, 1e-5) - ln64(x64 - h * u, w1, b, 1e-5)) / (2 * h) * dy64).sum()
    assert abs(fd - (dx.astype(np.float64) * u).sum()) < 1e-3 * max(1.0, abs(fd))
    # general gamma: the reference's closed form; dweight still the true gradient
    w = RNG.normal(1, 0.2, n).astype(np.float32)
    _, mean, rstd = orc.layer_norm_train(x, w, b, 1e-5, block)
    dx, dw, db = orc.layer_norm_backward(dy, x, w, mean, rstd, None, None, block)
    assert rel_inf(dx, ln_ref_formula64(dy, x, w, 1e-5)) < 1e-4
    xt, wt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w))
    torch.nn.functional.layer_norm(xt, (n,), wt, None, 1e-5).backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dw, wt.grad.numpy()) < 1e-4


def test_layernorm_backward_sensitivity(orc):
    # dropping the c2 (variance) term of dx must fail
    m, n = 4, 64
    x = RNG.normal(0, 1, (m, n)).astype(np.float32)
    w, dy = np.ones(n, np.float32), RNG.normal(0, 1, (m, n)).astype(np.float32)
    _, mean, rstd = orc.layer_norm_train(x, w, np.zeros(n, np.float32))
    dx, _, _ = orc.layer_norm_backward(dy, x, w, mean, rstd)
    c1 = (dy * w).mean(-1, keepdims=True)
    no_c2 = rstd[:, None] * w * (dy - c1)
    assert rel_inf(no_c2, dx) > 1e-2


@pytest.mark.parametrize("m,n,block", [(5, 128, 1024), (3, 1000, 256), (4, 37, 16)])
def test_rmsnorm_backward(orc, m, n, block):
    x = RNG.normal(0.3, 1.5, (m, n)).astype(np.float32)
    dy = RNG.normal(0, 1, (m, n)).astype(np.float32)
    dw0 = RNG.normal(0, 1, n).astype(np.float32)
    w1 = np.ones(n, np.float32)
    _, rrms = orc.rms_norm(x, w1, 1e-8, block)
    dx, dw = orc.rms_norm_backward(dy, x, w1, rrms, dw0, block)
    xt, wt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w1))
    (xt * torch.rsqrt((xt * xt).mean(-1, keepdim=True) + 1e-8) * wt).backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dx, xt.grad.numpy()) < 1e-4
    assert rel_inf(dw - dw0, wt.grad.numpy()) < 1e-4
    x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
    u = RNG.normal(0, 1, (m, n))
    h = 1e-6
    fd = ((rms64(x64 + h * u, w1, 1e-8) - rms64(x64 - h * u, w1, 1e-8)) / (2 * h) * dy64).sum()
    assert abs(fd - (dx.astype(np.float64) * u).sum()) < 1e-3 * max(1.0, abs(fd))
    w = RNG.normal(1, 0.2, n).astype(np.float32)
    _, rrms = orc.rms_norm(x, w, 1e-8, block)
    dx, dw = orc.rms_norm_backward(dy, x, w, rrms, None, block)
    assert rel_inf(dx, rms_ref_formula64(dy, x, w, 1e-8)) < 1e-4
    xt, wt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w))
    (xt * torch.rsqrt((xt * xt).mean(-1, keepdim=True) + 1e-8) * wt).backward(torch.tensor(dy, dtype=torch.float64))
    assert rel_inf(dw, wt.grad.numpy()) < 1e-4
