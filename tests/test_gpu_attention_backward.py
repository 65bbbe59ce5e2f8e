"""GPU parity of the attention backward (flash_attn2.rs:173-447) against the
reference fixture (tests/golden/flash_attn2/expected_backward_d*.bin) and the
CPU oracle: fp32 per-row kernels, the bf16 MFMA kernels (with and without a
stream workspace), causal masking, ragged lengths and grouped K/V heads."""
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


def oracle_forward(orc, q, k, v, scale, causal, group=1):
    """(o, l) with K/V heads shared by `group` consecutive query heads: the
    oracle runs on K/V repeated per query head."""
    kr, vr = np.repeat(k, group, axis=0), np.repeat(v, group, axis=0)
    o, l = orc.flash_attention(q, kr, vr, scale, causal)
    return o, l


def backward_ref(orc, q, k, v, o, do, l, scale, causal, group=1):
    """(dq, dk, dv); dk/dv of a shared K/V head sum over its query heads."""
    kr, vr = np.repeat(k, group, axis=0), np.repeat(v, group, axis=0)
    dq, dk, dv = orc.flash_attention_backward(q, kr, vr, o, do, l, scale, causal)
    bhk = k.shape[0]
    return dq, dk.reshape(bhk, group, *dk.shape[1:]).sum(1), dv.reshape(bhk, group, *dv.shape[1:]).sum(1)


def check_grad(buf, ref, what):
    """bf16 gradient: the element-wise bf16 bound and a norm-wise 8e-3."""
    bits = buf.to_host()
    ea = check_bf16(bits, ref, what)
    er = check_bf16_normwise(bits, ref, what)
    print(f"  {what}: max abs err {ea:.3g}, norm-wise {er:.3g}, max |ref| {float(np.max(np.abs(ref))):.3g}",
          flush=True)


@pytest.mark.parametrize("entry", ["split", "combined"])
def test_f32_fixture(dev, orc, entry):
    shape = (4, 8, 64)
    q, k, v, do = (load_golden(f"flash_attn2/{n}.bin").reshape(shape) for n in ("q", "k", "v", "do"))
    o = load_golden("flash_attn2/expected_forward_o.bin").reshape(shape)
    l = load_golden("flash_attn2/expected_forward_l.bin").reshape(4, 8)
    b = [dev.upload(a) for a in (q, k, v, o, do, l)]
    if entry == "split":
        dq = K.flash_attention_backward_dq(*b, 0.125)
        dk, dv = K.flash_attention_backward_dkv(*b, 0.125)
    else:
        dq, dk, dv = K.attention_backward(*b, softmax_scale=0.125)
    rq, rk, rv = orc.flash_attention_backward(q, k, v, o, do, l, 0.125)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        g = got.to_host()
        # test_flash_attn2.rs backward bound, then the oracle
        assert np.max(np.abs(g - load_golden(f"flash_attn2/expected_backward_{name}.bin").reshape(shape))) < 1e-3
        check_f32(g, ref, name)


@pytest.mark.parametrize("bh,nq,nk,d,causal,group", [
    (2, 37, 37, 64, False, 1), (2, 37, 37, 64, True, 1), (3, 100, 130, 32, False, 1), (1, 64, 256, 128, True, 1),
    (2, 20, 53, 16, True, 1), (1, 70, 90, 256, False, 1), (4, 33, 41, 64, True, 2), (4, 25, 25, 32, False, 4)])
def test_f32_vs_oracle(dev, orc, bh, nq, nk, d, causal, group):
    rng = np.random.default_rng(bh * 1009 + nq * 31 + nk)
    q = rng.normal(0, 1, (bh, nq, d)).astype(np.float32)
    k = rng.normal(0, 1, (bh // group, nk, d)).astype(np.float32)
    v = rng.normal(0, 1, (bh // group, nk, d)).astype(np.float32)
    do = rng.normal(0, 1, (bh, nq, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    o, l = oracle_forward(orc, q, k, v, scale, causal, group)
    rq, rk, rv = backward_ref(orc, q, k, v, o, do, l, scale, causal, group)
    print(f"[attn bwd f32] bh={bh} nq={nq} nk={nk} d={d} causal={causal} group={group}", flush=True)
    b = [dev.upload(a) for a in (q, k, v, o, do, l)]
    dq, dk, dv = K.attention_backward(*b, q_heads=group, kv_heads=1, causal=causal)
    check_f32(dq.to_host(), rq, "dq")
    check_f32(dk.to_host(), rk, "dk")
    check_f32(dv.to_host(), rv, "dv")
    if group == 1:
        dq2 = K.flash_attention_backward_dq(*b, causal=causal).to_host()
        dk2, dv2 = K.flash_attention_backward_dkv(*b, causal=causal)
        np.testing.assert_array_equal(dq2, dq.to_host())
        np.testing.assert_array_equal(dk2.to_host(), dk.to_host())
        np.testing.assert_array_equal(dv2.to_host(), dv.to_host())


BF16_CASES = [  # bh, nq, nk, d, causal, group
    (2, 128, 128, 128, False, 1),
    (2, 128, 128, 128, True, 1),
    (3, 200, 77, 64, False, 1),
    (2, 77, 300, 64, True, 1),
    (1, 513, 513, 128, True, 1),
    (2, 96, 160, 128, False, 1),
    (4, 130, 130, 64, True, 2),
    (8, 64, 200, 128, False, 4),
    # head_dim 128 on the two-workgroup dK/dV kernel (32-row query tiles):
    # causal with fewer queries than keys, and grouped causal at a ragged size
    (2, 77, 300, 128, True, 1),
    (4, 130, 130, 128, True, 2),
]


@pytest.mark.parametrize("bh,nq,nk,d,causal,group", BF16_CASES)
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_bf16_vs_oracle(dev, orc, bh, nq, nk, d, causal, group, scratch):
    rng = np.random.default_rng(bh * 7919 + nq * 13 + nk + d)
    q = rb(rng.normal(0, 1, (bh, nq, d)).astype(np.float32))
    k = rb(rng.normal(0, 1, (bh // group, nk, d)).astype(np.float32))
    v = rb(rng.normal(0, 1, (bh // group, nk, d)).astype(np.float32))
    do = rb(rng.normal(0, 1, (bh, nq, d)).astype(np.float32))
    scale = 1.0 / np.sqrt(d)
    o, l = oracle_forward(orc, q, k, v, scale, causal, group)
    o = rb(o)
    rq, rk, rv = backward_ref(orc, q, k, v, o, do, l, scale, causal, group)
    print(f"[attn bwd bf16] bh={bh} nq={nq} nk={nk} d={d} causal={causal} group={group} {scratch}", flush=True)
    b = [dev.upload(to_bf16(a), tg.bf16) for a in (q, k, v, o, do)] + [dev.upload(l)]

    def run():
        out = K.attention_backward(*b, q_heads=group, kv_heads=1, causal=causal)
        split = None
        if group == 1:
            split = (K.flash_attention_backward_dq(*b, causal=causal),) + K.flash_attention_backward_dkv(
                *b, causal=causal)
        dev.synchronize()
        return out, split

    if scratch == "workspace":
        with stream_workspace(dev, K.attention_backward_workspace_size(bh // group, group, nq)):
            out, split = run()
    else:
        out, split = run()
    for name, got, ref in zip(("dq", "dk", "dv"), out, (rq, rk, rv)):
        check_grad(got, ref, name)
    if split is not None:
        for name, got, ref in zip(("dq", "dk", "dv"), split, (rq, rk, rv)):
            check_grad(got, ref, "split " + name)


def test_bf16_training_shape(dev, orc):
    # B=2, H=8, S=1024, D=128 causal: one forward on the GPU, its o / lse fed
    # to the backward, everything checked against the oracle in full
    bh, s, d = 16, 1024, 128
    rng = np.random.default_rng(0x7EE70003)
    q, k, v, do = (rb(rng.standard_normal((bh, s, d), dtype=np.float32)) for _ in range(4))
    print(f"[attn bwd bf16] training shape bh={bh} s={s} d={d} causal", flush=True)
    qb, kb, vb, dob = (dev.upload(to_bf16(a), tg.bf16) for a in (q, k, v, do))
    lse = tg.Buffer(tg.f32, (bh, s))
    ob = K.flash_attention(qb, kb, vb, causal=True, lse=lse)
    o = from_bf16(ob.to_host()).reshape(bh, s, d)
    l = lse.to_host()
    ro, rl = orc.flash_attention(q, k, v, None, True)
    check_bf16(ob.to_host(), ro, "o")
    check_f32(l, rl, "lse", rel=1e-4)
    with stream_workspace(dev, K.attention_backward_workspace_size(bh, 1, s)):
        dq, dk, dv = K.attention_backward(qb, kb, vb, ob, dob, lse, causal=True)
        dev.synchronize()
    rq, rk, rv = orc.flash_attention_backward(q, k, v, o, do, l, None, True)
    check_grad(dq, rq, "dq")
    check_grad(dk, rk, "dk")
    check_grad(dv, rv, "dv")


def test_no_queries_gives_zero_dkv(dev):
    k = dev.upload(np.ones((2, 5, 32), np.float32))
    q = tg.Buffer(tg.f32, (2, 1, 32))  # never read: n_ctx_q = 0
    dk, dv = tg.Buffer(tg.f32, (2, 5, 32)), tg.Buffer(tg.f32, (2, 5, 32))
    for buf in (dk, dv):
        buf.to_device(np.full((2, 5, 32), 7.0, np.float32))
    import ctypes
    from teenygrad_amd import _lib
    tg.check(_lib.lib.teeny_flash_attention2_backward_dkv(q.ptr, k.ptr, k.ptr, q.ptr, q.ptr, q.ptr, dk.ptr, dv.ptr,
                                                         0, 5, ctypes.c_float(0.1), 2, 32, 0, _lib.F32, None))
    np.testing.assert_array_equal(dk.to_host(), 0.0)
    np.testing.assert_array_equal(dv.to_host(), 0.0)


@pytest.mark.parametrize("d", [16, 32, 256])
def test_bf16_forward_then_backward_small_and_large_heads(dev, orc, d):
    # bf16 at head sizes off the matrix-core kernels: the GPU forward's own O
    # and L feed the GPU backward, as a lowered training graph runs them
    bh, nq, nk, causal = 3, 90, 120, True
    rng = np.random.default_rng(d)
    q = rb(rng.normal(0, 1, (bh, nq, d)).astype(np.float32))
    k = rb(rng.normal(0, 1, (bh, nk, d)).astype(np.float32))
    v = rb(rng.normal(0, 1, (bh, nk, d)).astype(np.float32))
    do = rb(rng.normal(0, 1, (bh, nq, d)).astype(np.float32))
    scale = 1.0 / np.sqrt(d)
    print(f"[attn fwd+bwd bf16] d={d}", flush=True)
    qb, kb, vb, dob = (dev.upload(to_bf16(a), tg.bf16) for a in (q, k, v, do))
    lse = tg.Buffer(tg.f32, (bh, nq))
    ob = K.flash_attention(qb, kb, vb, scale, causal, lse=lse)
    o_ref, l_ref = oracle_forward(orc, q, k, v, scale, causal, 1)
    check_bf16(ob.to_host(), o_ref, "o")
    assert np.max(np.abs(lse.to_host() - l_ref)) < 1e-3
    dq, dk, dv = K.attention_backward(qb, kb, vb, ob, dob, lse, q_heads=1, kv_heads=1, causal=causal)
    rq, rk, rv = backward_ref(orc, q, k, v, rb(o_ref), do, l_ref, scale, causal, 1)
    for name, got, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), (rq, rk, rv)):
        check_grad(got, ref, name)
