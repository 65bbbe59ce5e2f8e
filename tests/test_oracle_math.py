"""Pins the CPU oracle where the reference's fixtures leave it open.

Each check compares the oracle (a restatement of the reference kernels'
loops) with an independent formulation — a float64 closed form, a
brute-force loop, numpy's own reductions, torch's CPU SDPA — on shapes the
fixtures do not cover (ragged tiles, strides, padding, groups, causal
masking, nq != nk).  The `*_sensitivity` tests show each check rejects a
plausible mistake (wrong sign, transposed operand, dropped term) planted on
the CPU side.
"""
import numpy as np
import pytest

RNG = np.random.default_rng(1234)


def rel_inf(got, want):
    """Norm-wise relative error ||got - want||_inf / ||want||_inf."""
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


# ── activations ─────────────────────────────────────────────────────────────


def gelu_tanh64(x):
    """0.5 x (1 + tanh(z)) == x * sigmoid(2z), z = sqrt(2/pi) (x + 0.044715 x^3); the
    sigmoid form avoids 1 + tanh(z) cancelling for z << 0.  float64, scipy's expit."""
    from scipy.special import expit
    x = x.astype(np.float64)
    return x * expit(2.0 * np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3))


def silu64(x):
    from scipy.special import expit
    x = x.astype(np.float64)
    return x * expit(x)


def test_activation_closed_forms(orc):
    x = np.concatenate([RNG.normal(0, 3, 5000), [0.0, -0.0, 80.0, -80.0, 1e-30, -1e-30]]).astype(np.float32)
    np.testing.assert_array_equal(orc.relu(x, block_size=1024), np.maximum(x, 0))
    # elementwise relative bound with an absolute floor for values near 0
    for fn, ref in ((orc.gelu, gelu_tanh64), (orc.silu, silu64)):
        got = fn(x, block_size=1024).astype(np.float64)
        want = ref(x)
        assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-30), fn.__name__


def test_activation_gradients_vs_finite_differences(orc):
    # d/dx of the float64 closed forms by central differences (truncation error ~h^2 = 1e-12):
    # a dropped term, a wrong sign or a wrong constant in the restated derivative fails this
    x = np.concatenate([RNG.normal(0, 2.5, 4000), [0.0, -0.0, 6.0, -6.0, 30.0, -30.0]])
    x32 = x.astype(np.float32)
    dy = RNG.normal(0, 1, x.size).astype(np.float32)
    h = 1e-6
    xd = x32.astype(np.float64)
    for fn, ref in ((orc.gelu_backward, gelu_tanh64), (orc.silu_backward, silu64)):
        want = dy.astype(np.float64) * (ref(xd + h) - ref(xd - h)) / (2 * h)
        got = fn(dy, x32, block_size=1024).astype(np.float64)
        assert np.all(np.abs(got - want) <= 2e-6 * np.abs(dy) + 1e-5 * np.abs(want)), fn.__name__


def test_activation_gradients_linear_in_dy_and_relu_mask(orc):
    x = RNG.normal(0, 2, 3000).astype(np.float32)
    dy = RNG.normal(0, 1, 3000).astype(np.float32)
    for fn in (orc.gelu_backward, orc.silu_backward):
        # scaling dy by 2 scales dx by 2 exactly (one rounding of the same product)
        np.testing.assert_array_equal(fn(2 * dy, x), 2 * fn(dy, x))
    y = np.maximum(x, 0)
    y[:3] = [0.0, np.nan, -0.0]
    got = orc.relu_backward(dy, y)
    np.testing.assert_array_equal(got[3:], np.where(y[3:] > 0, dy[3:], 0))
    assert np.all(got[:3] == 0)  # y == 0, NaN and -0 select 0


def test_gelu_tanh_identity():
    # the tanh statement of the same function, where 1 + tanh does not cancel
    x = np.linspace(-4, 4, 1001)
    tanh_form = 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
    np.testing.assert_allclose(gelu_tanh64(x), tanh_form, rtol=1e-12, atol=1e-15)


def test_activation_program_range(orc):
    x = RNG.normal(0, 1, 4000).astype(np.float32)
    # only programs [1, 3) of BLOCK_SIZE 1024 run: elements 1024..3071
    y = orc.relu(x, block_size=1024, pid_begin=1, pid_end=3)
    assert np.all(y[:1024] == 0) and np.all(y[3072:] == 0)
    np.testing.assert_array_equal(y[1024:3072], np.maximum(x[1024:3072], 0))


def test_gelu_sensitivity(orc):
    # the exact-erf GELU differs from the tanh form by up to ~1e-3: the check must see it
    from math import erf
    x = np.linspace(-4, 4, 257).astype(np.float32)
    erf_gelu = np.array([0.5 * v * (1 + erf(v / np.sqrt(2))) for v in x.astype(np.float64)])
    assert np.max(np.abs(orc.gelu(x) - erf_gelu)) > 1e-4


# ── norms ───────────────────────────────────────────────────────────────────


@pytest.mark.parametrize("m,n,block", [(37, 300, 128), (4, 4096, 1024), (3, 1, 1024)])
def test_layernorm_closed_form(orc, m, n, block):
    x = RNG.normal(0.5, 2.0, (m, n)).astype(np.float32)
    w = RNG.normal(1, 0.1, n).astype(np.float32)
    b = RNG.normal(0, 0.1, n).astype(np.float32)
    x64 = x.astype(np.float64)
    mu = x64.mean(-1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(-1, keepdims=True)
    want = (x64 - mu) / np.sqrt(var + 1e-5) * w + b
    got = orc.layer_norm(x, w, b, eps=1e-5, block_n=block)
    assert rel_inf(got, want) < 1e-5


@pytest.mark.parametrize("m,n,block", [(37, 300, 128), (4, 4096, 1024)])
def test_rmsnorm_closed_form(orc, m, n, block):
    x = RNG.normal(0.5, 2.0, (m, n)).astype(np.float32)
    w = RNG.normal(1, 0.1, n).astype(np.float32)
    x64 = x.astype(np.float64)
    rr = 1.0 / np.sqrt((x64 ** 2).mean(-1) + 1e-8)
    y, r = orc.rms_norm(x, w, eps=1e-8, block_n=block)
    assert rel_inf(r, rr) < 1e-6
    assert rel_inf(y, x64 * rr[:, None] * w) < 1e-5


def test_layernorm_sensitivity(orc):
    # dropping beta, or using the unbiased variance, must fail the closed-form check
    x = RNG.normal(0, 1, (8, 64)).astype(np.float32)
    w = np.ones(64, np.float32)
    b = np.full(64, 0.25, np.float32)
    got = orc.layer_norm(x, w, b)
    x64 = x.astype(np.float64)
    mu = x64.mean(-1, keepdims=True)
    unbiased = (x64 - mu) / np.sqrt(x64.var(-1, ddof=1, keepdims=True) + 1e-5) + b
    no_beta = (x64 - mu) / np.sqrt(x64.var(-1, keepdims=True) + 1e-5)
    assert rel_inf(got, unbiased) > 1e-3 and rel_inf(got, no_beta) > 1e-3


# ── conv2d ──────────────────────────────────────────────────────────────────


def conv_brute(x, w, b, stride, pad, groups):
    """float64 loops over the zero-padded input (a different formulation from
    the oracle's masked strip loop)."""
    B, Cin, H, W = x.shape
    Cout, cg, KH, KW = w.shape
    sh, sw = stride
    ph, pw = pad
    xp = np.zeros((B, Cin, H + 2 * ph, W + 2 * pw))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    y = np.zeros((B, Cout, OH, OW))
    opg = Cout // groups
    for co in range(Cout):
        g = co // opg
        xs = xp[:, g * cg:(g + 1) * cg]
        for oh in range(OH):
            for ow in range(OW):
                patch = xs[:, :, oh * sh:oh * sh + KH, ow * sw:ow * sw + KW]
                y[:, co, oh, ow] = np.tensordot(patch, w[co].astype(np.float64), axes=3)
        if b is not None:
            y[:, co] += b[co]
    return y


CONV_CASES = [
    # B, Cin, Cout, H, W, KH, KW, stride, pad, groups
    (2, 3, 5, 9, 7, 3, 3, (1, 1), (1, 1), 1),
    (1, 4, 6, 11, 10, 3, 2, (2, 3), (1, 0), 2),
    (1, 6, 6, 8, 8, 3, 3, (1, 1), (1, 1), 6),   # depthwise
    (2, 8, 4, 7, 7, 1, 1, (2, 2), (0, 0), 1),   # strided 1x1 (downsample)
    (1, 3, 4, 16, 16, 7, 7, (2, 2), (3, 3), 1),  # stem-like
]


@pytest.mark.parametrize("case", CONV_CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_conv2d_brute_force(orc, case, with_bias):
    B, Cin, Cout, H, W, KH, KW, st, pd, G = case
    x = RNG.normal(0, 1, (B, Cin, H, W)).astype(np.float32)
    w = RNG.normal(0, 0.3, (Cout, Cin // G, KH, KW)).astype(np.float32)
    b = RNG.normal(0, 0.1, Cout).astype(np.float32) if with_bias else None
    want = conv_brute(x, w, b, st, pd, G)
    for block_ow in (4, 16):
        got = orc.conv2d_nchw(x, w, b, stride=st, padding=pd, groups=G, block_ow=block_ow)
        assert got.shape == want.shape
        assert rel_inf(got, want) < 1e-6


def test_conv2d_nhwc_is_transpose(orc):
    x = RNG.normal(0, 1, (2, 5, 6, 8)).astype(np.float32)  # NHWC
    w = RNG.normal(0, 0.3, (4, 3, 3, 8)).astype(np.float32)  # OHWI
    got = orc.conv2d_nhwc(x, w, None, stride=1, padding=1)
    want = conv_brute(x.transpose(0, 3, 1, 2), w.transpose(0, 3, 1, 2), None, (1, 1), (1, 1), 1)
    assert rel_inf(got, want.transpose(0, 2, 3, 1)) < 1e-6


@pytest.mark.parametrize("case", [(3, 9, 7, 5, 4, 3, 3, 1, 1), (2, 11, 11, 3, 6, 7, 7, 2, 3),
                                  (2, 6, 6, 8, 16, 1, 1, 2, 0)])
def test_conv2d_pixel_subset(orc, case):
    # the sampled-pixel API runs the same programs: bit-identical to the full run
    B, H, W, Cin, Cout, KH, KW, s, p = case
    x = RNG.normal(0, 1, (B, H, W, Cin)).astype(np.float32)
    w = RNG.normal(0, 0.3, (Cout, KH, KW, Cin)).astype(np.float32)
    b = RNG.normal(0, 0.1, Cout).astype(np.float32)
    full = orc.conv2d_nhwc(x, w, b, stride=s, padding=p)
    m = full.shape[0] * full.shape[1] * full.shape[2]
    pix = np.unique(np.concatenate([[0, m - 1], RNG.integers(0, m, 9)]))
    got = orc.conv2d_nhwc_pixels(x, w, pix, b, stride=s, padding=p)
    np.testing.assert_array_equal(got, full.reshape(m, Cout)[pix])
    with pytest.raises(ValueError):
        orc.conv2d_nhwc_pixels(x, w, [m], b, stride=s, padding=p)


def test_conv2d_sensitivity(orc):
    # a spatially flipped kernel (cross-correlation vs convolution) must fail
    x = RNG.normal(0, 1, (1, 2, 8, 8)).astype(np.float32)
    w = RNG.normal(0, 0.3, (3, 2, 3, 3)).astype(np.float32)
    got = orc.conv2d_nchw(x, w, None, padding=1)
    flipped = conv_brute(x, w[:, :, ::-1, ::-1].copy(), None, (1, 1), (1, 1), 1)
    assert rel_inf(got, flipped) > 1e-2


# ── attention ───────────────────────────────────────────────────────────────


def attn64(q, k, v, scale, causal):
    s = np.einsum("bqd,bkd->bqk", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        nq, nk = s.shape[1:]
        s = np.where(np.arange(nk)[None, :] > np.arange(nq)[:, None], -np.inf, s)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(-1, keepdims=True)
    return (p / l) @ v.astype(np.float64), (m + np.log(l))[..., 0]


@pytest.mark.parametrize("bh,nq,nk,d", [(3, 37, 37, 64), (2, 20, 53, 32), (1, 70, 16, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_closed_form(orc, bh, nq, nk, d, causal):
    q = RNG.normal(0, 1, (bh, nq, d)).astype(np.float32)
    k = RNG.normal(0, 1, (bh, nk, d)).astype(np.float32)
    v = RNG.normal(0, 1, (bh, nk, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    o, l = orc.flash_attention(q, k, v, scale, causal)
    wo, wl = attn64(q, k, v, scale, causal)
    assert rel_inf(o, wo) < 1e-5
    assert rel_inf(l, wl) < 1e-5


def test_attention_rows_subset(orc):
    q = RNG.normal(0, 1, (4, 33, 64)).astype(np.float32)
    k = RNG.normal(0, 1, (4, 33, 64)).astype(np.float32)
    v = RNG.normal(0, 1, (4, 33, 64)).astype(np.float32)
    o, l = orc.flash_attention(q, k, v, causal=True)
    rows = np.array([0, 5, 33, 131], dtype=np.int64)
    ro, rl = orc.flash_attention_rows(q, k, v, rows, causal=True)
    np.testing.assert_array_equal(ro, o.reshape(-1, 64)[rows])
    np.testing.assert_array_equal(rl, l.reshape(-1)[rows])


def test_attention_vs_torch_sdpa(orc):
    torch = pytest.importorskip("torch")
    q = RNG.normal(0, 1, (4, 50, 64)).astype(np.float32)
    k = RNG.normal(0, 1, (4, 50, 64)).astype(np.float32)
    v = RNG.normal(0, 1, (4, 50, 64)).astype(np.float32)
    for causal in (False, True):
        o, _ = orc.flash_attention(q, k, v, causal=causal)
        want = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), is_causal=causal).numpy()
        np.testing.assert_allclose(o, want, rtol=1e-5, atol=1e-5)


def test_attention_sensitivity(orc):
    # causal vs non-causal, and a transposed V, must both be caught
    q = RNG.normal(0, 1, (1, 16, 16)).astype(np.float32)
    k = RNG.normal(0, 1, (1, 16, 16)).astype(np.float32)
    v = RNG.normal(0, 1, (1, 16, 16)).astype(np.float32)
    o, _ = orc.flash_attention(q, k, v, causal=True)
    assert rel_inf(o, attn64(q, k, v, 0.25, False)[0]) > 1e-2
    assert rel_inf(o, attn64(q, k, v.transpose(0, 2, 1).copy(), 0.25, True)[0]) > 1e-2


# ── linear ──────────────────────────────────────────────────────────────────


def test_linear_closed_form(orc):
    x = RNG.normal(0, 1, (33, 70)).astype(np.float32)
    w = RNG.normal(0, 1, (17, 70)).astype(np.float32)
    b = RNG.normal(0, 1, 17).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert rel_inf(orc.linear(x, w, b), want) < 1e-5
    assert rel_inf(orc.linear(x, w, None), want - b) < 1e-5


def test_linear_backward_closed_form(orc):
    # dx = dy W, dw = dy^T x, db = column sums of dy, in float64; a transposed
    # operand or a dropped bias gradient fails
    x = RNG.normal(0, 1, (37, 50)).astype(np.float32)
    w = RNG.normal(0, 1, (23, 50)).astype(np.float32)
    dy = RNG.normal(0, 1, (37, 23)).astype(np.float32)
    x64, w64, dy64 = (a.astype(np.float64) for a in (x, w, dy))
    dx, dw, db = orc.linear_backward(x, w, dy)
    assert rel_inf(dx, dy64 @ w64) < 1e-5
    assert rel_inf(dw, dy64.T @ x64) < 1e-5
    assert rel_inf(db, dy64.sum(axis=0)) < 1e-5
    # sensitivity: the forward's own contraction (x W^T) and a dw without the
    # transpose of dy have different values
    assert rel_inf(dw, (dy64.T @ x64)[::-1]) > 1e-2
    assert rel_inf(db, dy64.sum(axis=1)[:23]) > 1e-2
    # the gradient of the forward: <dy, linear(x + e dx_dir)> is linear in e
    e = RNG.normal(0, 1, x.shape)
    lhs = np.sum(dy64 * (e @ w64.T))
    assert abs(lhs - np.sum(dx * e)) <= 1e-4 * abs(lhs) + 1e-6
