"""GPU parity: flash attention (fp32 reference-structured kernel and the bf16
MFMA kernel) against the reference fixture and the CPU oracle."""
import math

import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from gpu_util import check_bf16, check_f32
from teenygrad_amd import kernels as K
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def test_f32_fixture(dev, orc):
    q = load_golden("flash_attn2/q.bin").reshape(4, 8, 64)
    k = load_golden("flash_attn2/k.bin").reshape(4, 8, 64)
    v = load_golden("flash_attn2/v.bin").reshape(4, 8, 64)
    lse = tg.Buffer(tg.f32, (4, 8))
    o = K.flash_attention(dev.upload(q), dev.upload(k), dev.upload(v), 0.125, lse=lse).to_host()
    # test_flash_attn2.rs:165,174
    assert np.max(np.abs(o - load_golden("flash_attn2/expected_forward_o.bin").reshape(4, 8, 64))) < 1e-4
    assert np.max(np.abs(lse.to_host() - load_golden("flash_attn2/expected_forward_l.bin").reshape(4, 8))) < 1e-4
    oo, ol = orc.flash_attention(q, k, v, 0.125)
    check_f32(o, oo, "o")
    check_f32(lse.to_host(), ol, "lse")


@pytest.mark.parametrize("bh,nq,nk,d,causal", [
    (2, 37, 37, 64, False), (2, 37, 37, 64, True), (3, 100, 130, 32, False),
    (1, 64, 256, 128, True), (2, 20, 53, 16, True), (1, 70, 200, 256, False)])
def test_f32_vs_oracle(dev, orc, bh, nq, nk, d, causal):
    rng = np.random.default_rng(bh * 7 + nq)
    q = rng.normal(0, 1, (bh, nq, d)).astype(np.float32)
    k = rng.normal(0, 1, (bh, nk, d)).astype(np.float32)
    v = rng.normal(0, 1, (bh, nk, d)).astype(np.float32)
    lse = tg.Buffer(tg.f32, (bh, nq))
    o = K.flash_attention(dev.upload(q), dev.upload(k), dev.upload(v), causal=causal, lse=lse).to_host()
    oo, ol = orc.flash_attention(q, k, v, causal=causal)
    check_f32(o, oo, "o")
    check_f32(lse.to_host(), ol, "lse")


def bf16_inputs(rng, bh, nq, nk, d):
    q = from_bf16(to_bf16(rng.standard_normal((bh, nq, d), dtype=np.float32)))
    k = from_bf16(to_bf16(rng.standard_normal((bh, nk, d), dtype=np.float32)))
    v = from_bf16(to_bf16(rng.standard_normal((bh, nk, d), dtype=np.float32)))
    return q, k, v


def run_bf16(dev, q, k, v, causal):
    bh, nq, d = q.shape
    lse = tg.Buffer(tg.f32, (bh, nq))
    o = K.flash_attention(dev.upload(to_bf16(q), tg.bf16), dev.upload(to_bf16(k), tg.bf16),
                          dev.upload(to_bf16(v), tg.bf16), 1.0 / math.sqrt(d), causal, lse=lse)
    return o.to_host(), lse.to_host()


@pytest.mark.parametrize("bh,nq,nk,d,causal", [
    (2, 128, 128, 128, False), (2, 128, 128, 128, True), (3, 200, 200, 128, True),
    (2, 100, 300, 64, False), (1, 257, 129, 128, True), (4, 64, 64, 64, True),
    (1, 1000, 1000, 128, True), (2, 300, 77, 128, False), (1, 512, 512, 64, False),
    (1, 33, 17, 128, False), (2, 70, 5, 64, True), (1, 130, 190, 64, True),
    # head sizes off the matrix-core kernel (the per-row kernel, as the
    # reference takes any HEAD_DIM, flash_attn2.rs:53)
    (2, 100, 130, 16, True), (3, 70, 70, 32, False), (1, 129, 200, 32, True), (2, 65, 90, 256, False),
    (1, 140, 140, 256, True)])
def test_bf16_vs_oracle(dev, orc, bh, nq, nk, d, causal):
    print(f"[attn bf16] bh={bh} nq={nq} nk={nk} d={d} causal={causal}", flush=True)
    q, k, v = bf16_inputs(np.random.default_rng(nq * 31 + nk), bh, nq, nk, d)
    o, lse = run_bf16(dev, q, k, v, causal)
    oo, ol = orc.flash_attention(q, k, v, causal=causal)
    check_bf16(o, oo, "o")
    assert np.max(np.abs(lse - ol)) < 1e-3


@pytest.mark.parametrize("scale,causal", [(-0.125, False), (-0.0625, True), (0.0, False), (0.0, True),
                                          (0.5, True)])
def test_bf16_scale(dev, orc, scale, causal):
    # a negative scale is applied by negating Q inside the kernel; a zero scale
    # gives uniform weights over the unmasked keys
    bh, nq, nk, d = 2, 150, 150, 128
    print(f"[attn bf16 scale] scale={scale} causal={causal}", flush=True)
    q, k, v = bf16_inputs(np.random.default_rng(77), bh, nq, nk, d)
    lse = tg.Buffer(tg.f32, (bh, nq))
    o = K.flash_attention(dev.upload(to_bf16(q), tg.bf16), dev.upload(to_bf16(k), tg.bf16),
                          dev.upload(to_bf16(v), tg.bf16), scale, causal, lse=lse).to_host()
    oo, ol = orc.flash_attention(q, k, v, softmax_scale=scale, causal=causal)
    check_bf16(o, oo, "o")
    assert np.max(np.abs(lse.to_host() - ol)) < 1e-3


@pytest.mark.parametrize("s,causal", [(2048, True), (4096, False)])
def test_bf16_config(dev, orc, s, causal):
    # causal S=2048 and non-causal S=4096, B*H = 8*32, D = 128: the whole
    # output (every row of every head) and every LSE entry against the oracle
    bh, d = 256, 128
    print(f"[attn bf16 config] BH={bh} S={s} causal={causal}", flush=True)
    q, k, v = bf16_inputs(np.random.default_rng(0x7EE70002 + s), bh, s, s, d)
    o, lse = run_bf16(dev, q, k, v, causal)
    oo, ol = orc.flash_attention(q, k, v, causal=causal)
    print(f"[attn bf16 config] oracle done, comparing {o.size} outputs", flush=True)
    for h0 in range(0, bh, 32):  # in head blocks, to bound the float64 temporaries
        check_bf16(o[h0:h0 + 32], oo[h0:h0 + 32], f"o heads {h0}..{h0 + 31}")
    assert np.max(np.abs(lse - ol)) < 1e-3
