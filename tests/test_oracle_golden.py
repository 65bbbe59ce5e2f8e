"""Pins the CPU oracle to the reference's own golden fixtures.

The fixtures under tests/golden/ are copied byte-for-byte from
kernels/teeny-kernels/tests/fixtures/ (written by that directory's
generate.py with torch.manual_seed(42)); the tolerances are the reference's
own assertions for the same fixtures.
"""
import numpy as np
import pytest

from conftest import load_golden


@pytest.mark.parametrize("op,tol", [("relu", 0.0), ("gelu", 2e-5), ("silu", 1e-5)])
def test_activations_match_fixture(orc, op, tol):
    # relu: test_relu.rs:98 (exact); gelu: test_gelu.rs:108 (2e-5); silu: test_sigmoid.rs:224 (1e-5)
    x = load_golden(f"{op}/x.bin")
    want = load_golden(f"{op}/expected_forward.bin")
    got = getattr(orc, op)(x)
    assert x.size == 1024
    np.testing.assert_allclose(got, want, rtol=0, atol=tol)


@pytest.mark.parametrize("op,tol", [("relu", 0.0), ("gelu", 2e-5), ("silu", 1e-5)])
def test_activation_backward_matches_fixture(orc, op, tol):
    # relu: test_relu.rs:148 (exact, on the forward OUTPUT y_backward.bin);
    # gelu: test_gelu.rs:157 (2e-5); silu: test_sigmoid.rs:274 (1e-5)
    if op == "relu":
        dy, saved = load_golden("relu/dy_backward.bin"), load_golden("relu/y_backward.bin")
    else:
        dy, saved = load_golden(f"{op}/dy.bin"), load_golden(f"{op}/x.bin")
    want = load_golden(f"{op}/expected_backward.bin")
    got = getattr(orc, f"{op}_backward")(dy, saved)
    assert dy.size == 1024
    np.testing.assert_allclose(got, want, rtol=0, atol=tol)


def test_layernorm_matches_fixture(orc):
    # test_layernorm.rs:159 — 16 x 128, eps 1e-5, |d| < 1e-4
    x = load_golden("layernorm/x.bin").reshape(16, 128)
    w = load_golden("layernorm/weight.bin")
    b = load_golden("layernorm/bias.bin")
    want = load_golden("layernorm/expected_forward.bin").reshape(16, 128)
    got = orc.layer_norm(x, w, b, eps=1e-5, block_n=1024)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4)
    # the reference launches BLOCK_N=1024 from the lowering; a BLOCK_N smaller than
    # the row (3 passes over 4 tiles) must agree too
    got32 = orc.layer_norm(x, w, b, eps=1e-5, block_n=32)
    np.testing.assert_allclose(got32, want, rtol=0, atol=1e-4)


def test_rmsnorm_matches_fixture(orc):
    # test_rmsnorm.rs:144,152 — 16 x 128, eps 1e-8, y and rrms within 1e-4
    x = load_golden("rmsnorm/x.bin").reshape(16, 128)
    w = load_golden("rmsnorm/weight.bin")
    want_y = load_golden("rmsnorm/expected_forward.bin").reshape(16, 128)
    want_r = load_golden("rmsnorm/expected_rrms.bin")
    y, r = orc.rms_norm(x, w, eps=1e-8)
    np.testing.assert_allclose(y, want_y, rtol=0, atol=1e-4)
    np.testing.assert_allclose(r, want_r, rtol=0, atol=1e-4)


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_conv2d_matches_fixture(orc, case, pad, oh):
    # test_conv2d.rs:203 — B=1, Cin=2, Cout=4, 8x8, 3x3, |d| < 1e-4
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    want = load_golden(f"{case}/expected_forward.bin").reshape(1, 4, oh, oh)
    for block_ow in (8, 16):
        got = orc.conv2d_nchw(x, w, padding=pad, block_ow=block_ow)
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-4)


def test_flash_attention_matches_fixture(orc):
    # test_flash_attn2.rs:165,174 — BH=4, N=8, D=64, scale 1/8, O and L within 1e-4
    q = load_golden("flash_attn2/q.bin").reshape(4, 8, 64)
    k = load_golden("flash_attn2/k.bin").reshape(4, 8, 64)
    v = load_golden("flash_attn2/v.bin").reshape(4, 8, 64)
    want_o = load_golden("flash_attn2/expected_forward_o.bin").reshape(4, 8, 64)
    want_l = load_golden("flash_attn2/expected_forward_l.bin").reshape(4, 8)
    o, l = orc.flash_attention(q, k, v, softmax_scale=1.0 / 8.0)
    np.testing.assert_allclose(o, want_o, rtol=0, atol=1e-4)
    np.testing.assert_allclose(l, want_l, rtol=0, atol=1e-4)


@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_matches_fixture(orc, with_bias):
    # test_linear.rs:48-54 — M=64, N=48, K=64, atol 0.1 + rtol 0.02 (the reference runs TF32)
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    b = load_golden("linear/bias.bin")
    want = load_golden(f"linear/expected_{'with' if with_bias else 'no'}_bias.bin").reshape(64, 48)
    got = orc.linear(x, w, b if with_bias else None)
    # fp32 accumulation is much tighter than the reference's TF32 bound
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-3)


def test_linear_backward_matches_fixture(orc):
    # test_linear.rs:434-626 — dx, dw, db against the committed fixtures
    # (M=64, N=48, K=64); the reference's bound is TF32-sized (atol 0.1 +
    # rtol 0.02), the fp32 oracle meets 1e-5 relative
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    dy = load_golden("linear/dy.bin").reshape(64, 48)
    dx, dw, db = orc.linear_backward(x, w, dy)
    for got, name, shape in ((dx, "dx", (64, 64)), (dw, "dw", (48, 64)), (db, "db", (48,))):
        want = load_golden(f"linear/expected_{name}.bin").reshape(shape)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * float(np.abs(want).max()), err_msg=name)
    _, _, none = orc.linear_backward(x, w, dy, use_bias=False)
    assert none is None
