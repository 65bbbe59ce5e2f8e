"""GPU parity: activations and norms against the fixtures and the CPU oracle."""
import ctypes

import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from gpu_util import check_bf16, check_f32, check_f32_elementwise
from teenygrad_amd import _lib, kernels as K
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu

M_CFG, N_CFG = 16384, 4096  # norm + activation workload: X[16384, 4096] bf16


@pytest.fixture(scope="module")
def x_cfg():
    """X ~ N(0,1), bf16-rounded; returns (bits, fp32 values)."""
    x = np.random.default_rng(0x7EE70001).standard_normal((M_CFG, N_CFG), dtype=np.float32)
    bits = to_bf16(x)
    return bits, from_bf16(bits).reshape(M_CFG, N_CFG)


@pytest.mark.parametrize("op,tol", [("relu", 0.0), ("gelu", 2e-5), ("silu", 1e-5)])
def test_act_f32_fixture(dev, orc, op, tol):
    x = load_golden(f"{op}/x.bin")
    want = load_golden(f"{op}/expected_forward.bin")
    got = getattr(K, op)(dev.upload(x)).to_host()
    assert np.max(np.abs(got - want)) <= tol
    check_f32_elementwise(got, getattr(orc, op)(x), op)


@pytest.mark.parametrize("op", ["relu", "gelu", "silu"])
def test_act_f32_ragged_and_unaligned(dev, orc, op):
    n = 10007
    x = np.random.default_rng(1).normal(0, 4, n + 1).astype(np.float32)
    xb = dev.upload(x)
    yb = tg.Buffer(tg.f32, (n + 1,))
    fn = getattr(_lib.lib, f"teeny_{op}_forward")
    # aligned, ragged tail (vector kernel + scalar tail)
    tg.check(fn(xb.ptr, yb.ptr, n, _lib.F32, None))
    check_f32_elementwise(yb.to_host()[:n], getattr(orc, op)(x[:n]), op)
    # 4-byte offset: not 16-byte aligned -> scalar kernel
    tg.check(fn(xb.ptr + 4, yb.ptr + 4, n, _lib.F32, None))
    check_f32_elementwise(yb.to_host()[1:], getattr(orc, op)(x[1:]), op + " unaligned")


def test_act_inplace(dev, orc):
    x = np.random.default_rng(2).normal(0, 2, 5000).astype(np.float32)
    b = dev.upload(x)
    K.silu(b, y=b)
    check_f32_elementwise(b.to_host(), orc.silu(x), "silu in place")


@pytest.mark.parametrize("op", ["relu", "gelu", "silu"])
def test_act_bf16_config(dev, orc, x_cfg, op):
    bits, xf = x_cfg
    print(f"[act bf16] {op} [{M_CFG}, {N_CFG}]", flush=True)
    y = getattr(K, op)(dev.upload(bits, tg.bf16)).to_host()
    check_bf16(y, getattr(orc, op)(xf), op)


@pytest.mark.parametrize("op,tol", [("relu", 0.0), ("gelu", 2e-5), ("silu", 1e-5)])
def test_act_backward_f32_fixture(dev, orc, op, tol):
    # the reference's backward fixtures and tolerances (test_relu.rs:148, test_gelu.rs:157,
    # test_sigmoid.rs:274); relu takes the forward output, gelu/silu the forward input
    if op == "relu":
        dy, saved = load_golden("relu/dy_backward.bin"), load_golden("relu/y_backward.bin")
    else:
        dy, saved = load_golden(f"{op}/dy.bin"), load_golden(f"{op}/x.bin")
    want = load_golden(f"{op}/expected_backward.bin")
    got = getattr(K, f"{op}_backward")(dev.upload(dy), dev.upload(saved)).to_host()
    assert np.max(np.abs(got - want)) <= tol
    check_f32(got, getattr(orc, f"{op}_backward")(dy, saved), f"{op}_backward f32")


def check_grad_f32(got, want, dy, what):
    """fp32 gradient parity: norm-wise relative 1e-5, and elementwise 1e-5 relative with an
    absolute floor of 2e-6 |dy|.  The derivative's terms are O(1) and cancel near its zero
    crossings (GELU near x = -0.75, SiLU near x = -1.28), where one fp32 rounding of a term
    (an FMA contraction, a 1-ulp exp) is a large relative error of the small result."""
    check_f32(got, want, what)
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - want.reshape(-1))
    bound = 1e-5 * np.abs(want.reshape(-1)) + 2e-6 * np.abs(dy.reshape(-1).astype(np.float64))
    assert np.all(err <= bound), f"{what}: {int((err > bound).sum())} elements beyond the bound"


@pytest.mark.parametrize("op", ["relu", "gelu", "silu"])
def test_act_backward_f32_ragged_unaligned_inplace(dev, orc, op):
    rng = np.random.default_rng(21)
    n = 100003  # vector body plus a scalar tail
    x = rng.normal(0, 3, n).astype(np.float32)
    dy = rng.normal(0, 1, n).astype(np.float32)
    saved = np.maximum(x, 0) if op == "relu" else x
    want = getattr(orc, f"{op}_backward")(dy, saved)
    fn = getattr(K, f"{op}_backward")
    check_grad_f32(fn(dev.upload(dy), dev.upload(saved)).to_host(), want, dy, f"{op} ragged")
    # pointers one element in: 4-byte aligned, not 16-byte aligned -> scalar kernel
    dyb = dev.upload(np.concatenate([[0], dy]).astype(np.float32))
    sb = dev.upload(np.concatenate([[0], saved]).astype(np.float32))
    dxb = tg.Buffer(tg.f32, (n + 1,))
    tg.check(getattr(_lib.lib, f"teeny_{op}_backward")(dyb.ptr + 4, sb.ptr + 4, dxb.ptr + 4, n,
                                                       _lib.F32, None))
    check_grad_f32(dxb.to_host()[1:], want, dy, f"{op} unaligned")
    # in place: dx written over dy
    d = dev.upload(dy)
    fn(d, dev.upload(saved), dx=d)
    check_grad_f32(d.to_host(), want, dy, f"{op} in place")


@pytest.mark.parametrize("op", ["relu", "gelu", "silu"])
def test_act_backward_bf16_config(dev, orc, x_cfg, op):
    bits, xf = x_cfg
    rng = np.random.default_rng(0x7EE70001 + 11)
    dyf = from_bf16(to_bf16(rng.standard_normal((M_CFG, N_CFG), dtype=np.float32)))
    savedf = from_bf16(to_bf16(np.maximum(xf, 0))) if op == "relu" else xf
    print(f"[act bwd bf16] {op} [{M_CFG}, {N_CFG}]", flush=True)
    got = getattr(K, f"{op}_backward")(dev.upload(to_bf16(dyf), tg.bf16),
                                        dev.upload(to_bf16(savedf), tg.bf16)).to_host()
    check_bf16(got, getattr(orc, f"{op}_backward")(dyf, savedf), f"{op}_backward bf16")


def test_layernorm_f32_fixture(dev, orc):
    x = load_golden("layernorm/x.bin").reshape(16, 128)
    w, b = load_golden("layernorm/weight.bin"), load_golden("layernorm/bias.bin")
    want = load_golden("layernorm/expected_forward.bin").reshape(16, 128)
    got = K.layer_norm(dev.upload(x), dev.upload(w), dev.upload(b), 1e-5).to_host()
    assert np.max(np.abs(got - want)) < 1e-4  # test_layernorm.rs:159
    check_f32(got, orc.layer_norm(x, w, b, 1e-5), "layernorm")


def test_rmsnorm_f32_fixture(dev, orc):
    x = load_golden("rmsnorm/x.bin").reshape(16, 128)
    w = load_golden("rmsnorm/weight.bin")
    rr = tg.Buffer(tg.f32, (16,))
    got = K.rms_norm(dev.upload(x), dev.upload(w), 1e-8, rrms=rr).to_host()
    assert np.max(np.abs(got - load_golden("rmsnorm/expected_forward.bin").reshape(16, 128))) < 1e-4
    assert np.max(np.abs(rr.to_host() - load_golden("rmsnorm/expected_rrms.bin"))) < 1e-4
    oy, orr = orc.rms_norm(x, w, 1e-8)
    check_f32(got, oy, "rmsnorm y")
    check_f32(rr.to_host(), orr, "rmsnorm rrms")


@pytest.mark.parametrize("m,n", [(37, 300), (5, 1), (3, 5000), (64, 4096), (9, 8200), (2, 20000),
                                 (20001, 256), (9001, 1000), (4500, 4096)])
def test_norms_f32_shapes(dev, orc, m, n):
    # register path (N % 4 == 0, N <= 4096), ragged rows, multi-pass path (N > 4096 or odd N);
    # the last three have more row blocks than fit on the chip at once, so each workgroup walks
    # several blocks (20001 rows of 256: four rows per block and a ragged last block)
    rng = np.random.default_rng(m * 1000 + n)
    x = rng.normal(0.3, 1.5, (m, n)).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    xb, wb, bb = dev.upload(x), dev.upload(w), dev.upload(b)
    check_f32(K.layer_norm(xb, wb, bb, 1e-5).to_host(), orc.layer_norm(x, w, b, 1e-5), "ln")
    rr = tg.Buffer(tg.f32, (m,))
    y = K.rms_norm(xb, wb, 1e-8, rrms=rr).to_host()
    oy, orr = orc.rms_norm(x, w, 1e-8)
    check_f32(y, oy, "rms y")
    check_f32(rr.to_host(), orr, "rms rrms")


@pytest.mark.parametrize("kind", ["layer", "rms"])
def test_norm_bf16_config(dev, orc, x_cfg, kind):
    bits, xf = x_cfg
    rng = np.random.default_rng(0x7EE70001 + 7)
    g = from_bf16(to_bf16(rng.normal(1, 0.02, N_CFG).astype(np.float32)))
    be = from_bf16(to_bf16(rng.normal(0, 0.02, N_CFG).astype(np.float32)))
    xb = dev.upload(bits, tg.bf16)
    gb, bb = dev.upload(to_bf16(g), tg.bf16), dev.upload(to_bf16(be), tg.bf16)
    print(f"[norm bf16] {kind} [{M_CFG}, {N_CFG}]", flush=True)
    if kind == "layer":
        y = K.layer_norm(xb, gb, bb, 1e-5).to_host()
        check_bf16(y, orc.layer_norm(xf, g, be, 1e-5), "layernorm bf16")
    else:
        rr = tg.Buffer(tg.f32, (M_CFG,))
        y = K.rms_norm(xb, gb, 1e-8, rrms=rr).to_host()
        oy, orr = orc.rms_norm(xf, g, 1e-8)
        check_bf16(y, oy, "rmsnorm bf16")
        check_f32(rr.to_host(), orr, "rrms")


@pytest.mark.parametrize("rms,act", [(False, "gelu"), (True, "silu"), (False, "relu"), (True, "gelu")])
def test_norm_act_fused_bf16(dev, orc, rms, act):
    rng = np.random.default_rng(11)
    m, n = 512, 4096
    xf = from_bf16(to_bf16(rng.standard_normal((m, n), dtype=np.float32)))
    g = from_bf16(to_bf16(rng.normal(1, 0.02, n).astype(np.float32)))
    be = from_bf16(to_bf16(rng.normal(0, 0.02, n).astype(np.float32)))
    y = K.norm_act(dev.upload(to_bf16(xf), tg.bf16), dev.upload(to_bf16(g), tg.bf16),
                   dev.upload(to_bf16(be), tg.bf16), 1e-8 if rms else 1e-5, rms, act).to_host()
    ref = orc.rms_norm(xf, g, 1e-8)[0] if rms else orc.layer_norm(xf, g, be, 1e-5)
    check_bf16(y, getattr(orc, act)(ref), f"fused {act}")
