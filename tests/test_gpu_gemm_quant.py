"""GPU parity: linear (fp32 / bf16), W8A16 GEMM and teeny-quant on the GPU."""
import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from gpu_util import check_bf16, check_f32, stream_workspace
from quant_cases import KNOWN
from teenygrad_amd import _lib, kernels as K
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def rb(a):
    return from_bf16(to_bf16(a))


@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_f32_fixture(dev, orc, with_bias):
    x = load_golden("linear/input.bin").reshape(64, 64)
    w = load_golden("linear/weight.bin").reshape(48, 64)
    b = load_golden("linear/bias.bin")
    want = load_golden(f"linear/expected_{'with' if with_bias else 'no'}_bias.bin").reshape(64, 48)
    got = K.linear(dev.upload(x), dev.upload(w), dev.upload(b) if with_bias else None).to_host()
    np.testing.assert_allclose(got, want, rtol=0.02, atol=0.1)  # test_linear.rs:48-54
    check_f32(got, orc.linear(x, w, b if with_bias else None), "linear f32")


def with_scratch(dev, scratch, need, fn):
    """Runs fn() with no stream workspace, or with one of ``need`` bytes."""
    if scratch == "workspace":
        if need == 0:
            pytest.skip("no scratch plan at this shape: same path as scratch=none")
        with stream_workspace(dev, need):
            return fn()
    return fn()


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (200, 300, 136), (64, 48, 64), (33, 17, 70), (256, 512, 1000),
                                   (64, 256, 4096), (96, 200, 3100)])
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_linear_bf16(dev, orc, m, n, k, scratch):
    # (64, 256, 4096) splits along K given a workspace; (33, 17, 70) and
    # (96, 200, 3100) have K % 8 != 0 and take the generic kernel
    rng = np.random.default_rng(m + n + k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb((rng.standard_normal((n, k), dtype=np.float32) / np.sqrt(k)).astype(np.float32))
    b = rb(rng.normal(0, 0.5, n).astype(np.float32))
    need = K.linear_workspace_size(m, n, k, tg.bf16)
    if dev.info()["compute_units"] == 256:
        assert (need > 0) == ((m, n, k) == (64, 256, 4096)), need
    got = with_scratch(dev, scratch, need, lambda: K.linear(
        dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16), dev.upload(to_bf16(b), tg.bf16)).to_host())
    check_bf16(got, orc.linear(x, w, b), "linear bf16")


@pytest.mark.parametrize("m,n,k", [(16421, 64, 128), (16384, 128, 256), (20000, 256, 64)])
def test_linear_bf16_stream(dev, orc, m, n, k):
    # M >= 16384 with K, N in {64, 128, 256}: the streaming kernel (B staged
    # once per workgroup, 32-row blocks per wave; 16421 and 20000 end in a
    # partial block)
    rng = np.random.default_rng(m + n + k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb((rng.standard_normal((n, k), dtype=np.float32) / np.sqrt(k)).astype(np.float32))
    b = rb(rng.normal(0, 0.5, n).astype(np.float32))
    assert K.linear_workspace_size(m, n, k, tg.bf16) == 0
    got = K.linear(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16),
                   dev.upload(to_bf16(b), tg.bf16)).to_host()
    check_bf16(got, orc.linear(x, w, b), "linear bf16 stream")


@pytest.mark.parametrize("pad,offset", [(8, 0), (4, 0), (0, 8), (8, 16)])
def test_linear_bf16_stream_padded_rows(dev, orc, pad, offset):
    # the reference's LinearForward passes output_row_stride as stride_ym
    # (linear.rs:297-311), which may be padded; M = 16421 with K = 128, N = 64 is
    # a streaming shape.  Row pitch N + pad and y offset by `offset` bytes: the
    # streaming kernel takes 16-byte aligned rows (pad 8, offset 0 or 16), the
    # tiled kernels the rest; padding columns and the bytes before y stay untouched
    m, n, k = 16421, 64, 128
    print(f"[linear stream padded] ldy={n + pad} offset={offset}", flush=True)
    rng = np.random.default_rng(pad + offset)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb((rng.standard_normal((n, k), dtype=np.float32) / np.sqrt(k)).astype(np.float32))
    xb, wb = dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16)
    ldy = n + pad
    sentinel = np.uint16(0x7FC1)  # a NaN pattern no result has
    ybuf = dev.upload(np.full(offset // 2 + m * ldy, sentinel, np.uint16), tg.bf16)
    tg.check(_lib.lib.teeny_linear_forward(xb.ptr, wb.ptr, None, ybuf.ptr + offset, m, n, k, k, 1, k, 1,
                                           ldy, 1, _lib.BF16, None))
    host = ybuf.to_host()
    assert np.all(host[:offset // 2] == sentinel)
    y = host[offset // 2:].reshape(m, ldy)
    assert np.all(y[:, n:] == sentinel)
    rows = np.concatenate([np.arange(0, 64), np.arange(0, m, 97), np.arange(m - 64, m)])
    check_bf16(y[rows, :n], orc.linear(x[rows], w), f"ldy={ldy} offset={offset}")


def tile_rows(m, tile, rng):
    """One row inside every `tile`-row block of [0, m), plus the first and last 64 rows."""
    starts = np.arange(0, m, tile, dtype=np.int64)
    pick = starts + (rng.random(starts.size) * np.minimum(tile, m - starts)).astype(np.int64)
    return np.unique(np.concatenate([np.arange(64), pick, np.arange(m - 64, m)]))


@pytest.mark.parametrize("m,n,k,pad", [(50000, 512, 128, 0), (50000, 512, 256, 8), (131072, 128, 384, 0),
                                       (40000, 1024, 512, 16), (12544, 1024, 256, 0), (12544, 512, 1024, 0),
                                       (20000, 384, 768, 8)])
def test_linear_bf16_persistent(dev, orc, m, n, k, pad):
    # >= 1.5 tiles of 128 x 128 per CU and 128 <= K <= 512 (<= 1024 for
    # N <= 1024): the persistent LDS-DMA kernel (one DMA ring per workgroup
    # across its tiles; 50000, 40000 and 20000 end in a partial row tile,
    # K = 128 is shorter than the ring; 12544 x 512 x 1024 and 20000 x 384
    # x 768 run 1.5-1.8 tiles per CU, some workgroups one tile).
    # Output rows padded to N + pad: the padding columns stay untouched.
    # One row of every 128-row tile (each workgroup's every tile) vs the oracle.
    print(f"[linear persistent] m={m} n={n} k={k} ldy={n + pad}", flush=True)
    rng = np.random.default_rng(m + n + k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb((rng.standard_normal((n, k), dtype=np.float32) / np.sqrt(k)).astype(np.float32))
    b = rb(rng.normal(0, 0.5, n).astype(np.float32))
    assert K.linear_workspace_size(m, n, k, tg.bf16) == 0
    xb, wb, bb = dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16), dev.upload(to_bf16(b), tg.bf16)
    ldy = n + pad
    sentinel = np.uint16(0x7FC1)
    ybuf = dev.upload(np.full(m * ldy, sentinel, np.uint16), tg.bf16)
    tg.check(_lib.lib.teeny_linear_forward(xb.ptr, wb.ptr, bb.ptr, ybuf.ptr, m, n, k, k, 1, k, 1, ldy, 1,
                                           _lib.BF16, None))
    y = ybuf.to_host().reshape(m, ldy)
    assert np.all(y[:, n:] == sentinel)
    assert np.all(np.isfinite(from_bf16(y[:, :n])))
    rows = tile_rows(m, 128, rng)
    check_bf16(y[rows, :n], orc.linear(x[rows], w, b), f"{rows.size} sampled rows")


def test_linear_bf16_large_tile(dev, orc):
    # 4096 x 512 x 4096: 256 x 256 tiles fill the chip -> large-tile kernel;
    # rows 0..31 and the last 32 rows against the oracle
    m, k, n = 4096, 512, 4096
    rng = np.random.default_rng(4096)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    w = rb(rng.normal(0, 0.05, (n, k)).astype(np.float32))
    y = K.linear(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16)).to_host()
    for lo, hi in ((0, 32), (m - 32, m)):
        check_bf16(y[lo:hi], orc.linear(x[lo:hi], w), f"rows {lo}..{hi}")


def test_linear_bf16_strided_generic(dev, orc):
    # x given as a transposed view (stride_xk = M): the generic kernel path
    rng = np.random.default_rng(3)
    m, n, k = 40, 24, 56
    xt = rb(rng.standard_normal((k, m), dtype=np.float32))  # x = xt^T
    w = rb((rng.standard_normal((n, k), dtype=np.float32) / 8).astype(np.float32))
    xb, wb = dev.upload(to_bf16(xt), tg.bf16), dev.upload(to_bf16(w), tg.bf16)
    y = tg.Buffer(tg.bf16, (m, n))
    tg.check(_lib.lib.teeny_linear_forward(xb.ptr, wb.ptr, None, y.ptr, m, n, k, 1, m, k, 1, n, 1,
                                           _lib.BF16, None))
    check_bf16(y.to_host(), orc.linear(np.ascontiguousarray(xt.T), w), "strided linear")


def quantized_weight(orc, rng, n, k):
    wf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    q, s, _, _ = orc.quantize_affine(wf, [n, k], "channel", 0)
    return q.reshape(n, k), s


@pytest.mark.parametrize("m,n,k,act", [(100, 200, 256, None), (256, 384, 512, "silu"),
                                       (64, 64, 4096, "gelu"), (37, 70, 40, "relu"), (5, 9, 48, None),
                                       (600, 96, 128, "relu"), (530, 200, 64, None)])
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_w8a16_small(dev, orc, m, n, k, act, scratch):
    # (37, 70, 40) and (5, 9, 48): K % 16 != 0 -> generic kernel; others MFMA;
    # given a workspace, (64, 64, 4096) splits along K
    rng = np.random.default_rng(m * n + k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    q, s = quantized_weight(orc, rng, n, k)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    need = K.linear_workspace_size(m, n, k, tg.i8)
    if dev.info()["compute_units"] == 256:
        assert (need > 0) == ((m, n, k) == (64, 64, 4096)), need
    got = with_scratch(dev, scratch, need, lambda: K.w8a16_linear(
        dev.upload(to_bf16(x), tg.bf16), dev.upload(q), dev.upload(s), dev.upload(bias), act=act).to_host())
    ref = orc.w8a16_linear(x, q, s, bias)
    if act is not None:
        ref = getattr(orc, act)(ref)
    check_bf16(got, ref, "w8a16")


_CONFIG_REF = {}


@pytest.mark.parametrize("scratch", ["none", "workspace"])
@pytest.mark.parametrize("k,n", [(4096, 11008), (11008, 4096)])
def test_w8a16_config(dev, orc, k, n, scratch):
    # M = 4096 tokens; weights N(0, 0.02) quantised per output channel on the GPU
    # (bit-exact with the oracle); the whole [M, N] output against the oracle
    m = 4096
    rng = np.random.default_rng(0x7EE70005 + k)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    wf = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    print(f"[w8a16 config] M={m} K={k} N={n} scratch={scratch}", flush=True)
    qg, sg, zg, _ = K.quantize_affine(dev.upload(wf), [n, k], "channel", 0)
    q, s, z, _ = orc.quantize_affine(wf, [n, k], "channel", 0)
    np.testing.assert_array_equal(qg.to_host().reshape(-1), q)
    np.testing.assert_array_equal(sg.to_host(), s)
    # the 256 x 256 LDS-DMA kernel converts the int8 weights in registers
    # ahead of each MFMA: no scratch, and an attached workspace changes nothing
    need = K.linear_workspace_size(m, n, k, tg.i8)
    assert need == 0, need
    need = 1 << 20
    y = with_scratch(dev, scratch, need, lambda: K.w8a16_linear(dev.upload(to_bf16(x), tg.bf16), qg, sg).to_host())
    if (k, n) not in _CONFIG_REF:  # one oracle run per shape, shared by both scratch modes
        _CONFIG_REF.clear()
        wdeq = orc.dequantize_affine(q, s, None, [n, k], "channel", 0)
        _CONFIG_REF[(k, n)] = orc.linear(x, wdeq)
    ref = _CONFIG_REF[(k, n)]
    for lo in range(0, m, 1024):
        check_bf16(y[lo:lo + 1024], ref[lo:lo + 1024], f"rows {lo}..{lo + 1023}")


# ── teeny-quant on the GPU: bit-exact with the oracle ──────────────────────


@pytest.mark.parametrize("case", KNOWN, ids=[c[0] for c in KNOWN])
def test_quant_known_answers(dev, case):
    name, data, shape, gran, axis, gs, sym, bits, want_q, want_s, want_z = case
    q, s, z, g = K.quantize_affine(dev.upload(np.array(data, np.float32)), shape, gran, axis, gs,
                                   sym, bits, want_groups=True)
    np.testing.assert_array_equal(q.to_host().reshape(-1), np.array(want_q, np.int8))
    np.testing.assert_array_equal(s.to_host(), np.array(want_s, np.float32))
    np.testing.assert_array_equal(z.to_host(), np.array(want_z, np.int32))


RANDOM = [((64, 96), "channel", 0, 1, True, 8), ((64, 96), "channel", 1, 1, True, 8),
          ((64, 96), "tensor", 0, 1, False, 8), ((8, 5, 33), "group", 2, 8, True, 8),
          ((8, 5, 33), "group", 1, 2, False, 4), ((8, 5, 33), "group", 0, 3, True, 4),
          ((256, 3, 3, 256), "channel", 0, 1, True, 8), ((3000, 17), "channel", 0, 1, False, 8),
          # contiguous groups split over several workgroups (rows of 40000 and a
          # 100003-element tensor), groups of 7 and 5 (quads straddling two
          # groups), and groups of 3 (the per-element kernel)
          ((5, 40000), "channel", 0, 1, True, 8), ((100003,), "tensor", 0, 1, False, 8),
          ((33, 7), "channel", 0, 1, True, 8), ((9, 5), "channel", 0, 1, False, 4), ((6, 3), "channel", 0, 1, True, 8)]


@pytest.mark.parametrize("shape,gran,axis,gs,sym,bits", RANDOM)
def test_quant_vs_oracle(dev, orc, shape, gran, axis, gs, sym, bits):
    x = np.random.default_rng(len(shape) + axis).normal(0, 0.02, shape).astype(np.float32)
    x.reshape(-1)[::5] *= 3.0
    q, s, z, g = K.quantize_affine(dev.upload(x), shape, gran, axis, gs, sym, bits, want_groups=True)
    oq, os_, oz, og = orc.quantize_affine(x, shape, gran, axis, gs, sym, bits)
    np.testing.assert_array_equal(g.to_host(), og)
    np.testing.assert_array_equal(s.to_host(), os_)
    np.testing.assert_array_equal(z.to_host(), oz)
    np.testing.assert_array_equal(q.to_host().reshape(-1), oq)
    d = K.dequantize_affine(q, s, z, shape, gran, axis, gs).to_host()
    np.testing.assert_array_equal(d.reshape(-1), orc.dequantize_affine(oq, os_, oz, shape, gran, axis, gs).reshape(-1))


def test_quant_empty_groups(dev):
    # shape [0, 4], per-channel over axis 1: 4 groups, no elements -> scale 1, zp = qmin (asym)
    ng = K.quant_num_groups([0, 4], "channel", 1)
    assert ng == 4
    x = tg.Buffer(tg.f32, (0,))
    q, s, z, _ = K.quantize_affine(x, [0, 4], "channel", 1, symmetric=False)
    np.testing.assert_array_equal(s.to_host(), np.ones(4, np.float32))
    np.testing.assert_array_equal(z.to_host(), np.full(4, -128, np.int32))
