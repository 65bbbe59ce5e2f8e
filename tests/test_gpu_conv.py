"""GPU parity: conv2d (fp32 direct, bf16 NHWC MFMA implicit GEMM, W8A16)."""
import numpy as np
import pytest

import teenygrad_amd as tg
from conftest import load_golden
from gpu_util import check_bf16, check_f32, stream_workspace
from teenygrad_amd import kernels as K
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def rb(a):
    return from_bf16(to_bf16(a))


@pytest.mark.parametrize("case,pad,oh", [("conv2d", 0, 6), ("conv2d_padded", 1, 8)])
def test_f32_fixture(dev, orc, case, pad, oh):
    x = load_golden(f"{case}/x.bin").reshape(1, 2, 8, 8)
    w = load_golden(f"{case}/w.bin").reshape(4, 2, 3, 3)
    want = load_golden(f"{case}/expected_forward.bin").reshape(1, 4, oh, oh)
    got = K.conv2d(dev.upload(x), dev.upload(w), padding=pad).to_host()
    assert np.max(np.abs(got - want)) < 1e-4  # test_conv2d.rs:203
    check_f32(got, orc.conv2d_nchw(x, w, padding=pad), "conv")


def test_f32_conv_bias_relu_config(dev, orc):
    # conv2d + bias + ReLU, fp32 NCHW, 1 x 64 -> 64, 56 x 56, 3 x 3, s1 p1
    rng = np.random.default_rng(0x7EE70000)
    x = rng.standard_normal((1, 64, 56, 56), dtype=np.float32)
    w = (rng.standard_normal((64, 64, 3, 3), dtype=np.float32) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = (rng.standard_normal(64, dtype=np.float32) * 0.01).astype(np.float32)
    got = K.conv2d(dev.upload(x), dev.upload(w), dev.upload(b), padding=1, act="relu").to_host()
    ref = orc.relu(orc.conv2d_nchw(x, w, b, padding=1))
    check_f32(got, ref, "conv+bias+relu")
    # unfused: the reference's two kernels
    y = K.conv2d(dev.upload(x), dev.upload(w), dev.upload(b), padding=1)
    check_f32(K.relu(y).to_host(), ref, "conv+bias then relu")


CASES = [
    # B, Cin, Cout, H, W, KH, KW, stride, pad, groups
    (2, 3, 5, 9, 7, 3, 3, (1, 1), (1, 1), 1),
    (1, 4, 6, 11, 10, 3, 2, (2, 3), (1, 0), 2),
    (1, 6, 6, 8, 8, 3, 3, (1, 1), (1, 1), 6),
    (2, 8, 4, 7, 7, 1, 1, (2, 2), (0, 0), 1),
    (1, 3, 4, 16, 16, 7, 7, (2, 2), (3, 3), 1),
    (1, 16, 12, 9, 9, 5, 5, (1, 1), (2, 2), 4),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("layout", ["nchw", "nhwc"])
def test_f32_cases(dev, orc, case, layout):
    B, Cin, Cout, H, W, KH, KW, st, pd, G = case
    rng = np.random.default_rng(Cin * 100 + Cout)
    x = rng.normal(0, 1, (B, Cin, H, W)).astype(np.float32)
    w = rng.normal(0, 0.3, (Cout, Cin // G, KH, KW)).astype(np.float32)
    b = rng.normal(0, 0.1, Cout).astype(np.float32)
    ref = orc.conv2d_nchw(x, w, b, stride=st, padding=pd, groups=G)
    if layout == "nchw":
        got = K.conv2d(dev.upload(x), dev.upload(w), dev.upload(b), st, pd, G).to_host()
    else:
        got = K.conv2d(dev.upload(np.ascontiguousarray(x.transpose(0, 2, 3, 1))),
                       dev.upload(np.ascontiguousarray(w.transpose(0, 2, 3, 1))), dev.upload(b), st,
                       pd, G, layout="nhwc").to_host().transpose(0, 3, 1, 2)
    check_f32(got, ref, f"{case} {layout}")


# fp32 NCHW 3x3 stride-1 convs with C_IN % 16 == 0 and W % 4 == 0, W <= 56:
# the row kernel (one output row x 16 output channels per workgroup)
ROW_CASES = [
    # B, Cin, Cout, H, W, pad (h, w), act, bias
    (2, 32, 40, 12, 12, (1, 1), "relu", True),   # ragged channel tile (40 = 2 x 16 + 8)
    (1, 16, 16, 8, 4, (0, 0), None, True),       # W = 4, no padding: OW = 2
    (3, 48, 20, 7, 56, (2, 4), "gelu", False),  # widest padding, OW = 62, Cout % 16 != 0
    (1, 64, 64, 56, 56, (1, 1), "silu", False),  # the 56 x 56 config without bias
    (2, 16, 8, 5, 52, (0, 3), None, True),       # H < KH + PH rows, one ragged tile only
]


@pytest.mark.parametrize("case", ROW_CASES)
def test_f32_nchw_row(dev, orc, case):
    B, Cin, Cout, H, W, pd, act, with_bias = case
    print(f"[conv f32 row] {case}", flush=True)
    rng = np.random.default_rng(Cin * 13 + Cout + W)
    x = rng.standard_normal((B, Cin, H, W), dtype=np.float32)
    w = (rng.standard_normal((Cout, Cin, 3, 3), dtype=np.float32) * np.sqrt(2.0 / (Cin * 9))).astype(np.float32)
    b = rng.normal(0, 0.1, Cout).astype(np.float32) if with_bias else None
    got = K.conv2d(dev.upload(x), dev.upload(w), dev.upload(b) if with_bias else None, 1, pd, act=act).to_host()
    ref = orc.conv2d_nchw(x, w, b, padding=pd)
    if act is not None:
        ref = getattr(orc, act)(ref)
    check_f32(got, ref, f"row {case}")
    # folded BatchNorm through the same kernel (per-channel scale before the shift)
    sc = rng.normal(1, 0.2, Cout).astype(np.float32)
    sh = rng.normal(0, 0.3, Cout).astype(np.float32)
    y = K.conv2d_bn_act(dev.upload(x), dev.upload(w), dev.upload(sc), dev.upload(sh), 1, pd, 1, "relu").to_host()
    c = orc.conv2d_nchw(x, w, None, padding=pd)
    check_f32(y, orc.relu(sc[None, :, None, None] * c + sh[None, :, None, None]), f"row+bn {case}")


BF16_CASES = [
    # B, Cin, Cout, H, W, KH, KW, stride, pad, act     (path)
    (2, 64, 64, 14, 14, 3, 3, 1, 1, "relu"),   # 3x3 implicit GEMM, 16-byte gather
    (2, 64, 256, 14, 14, 1, 1, 1, 0, None),    # 1x1 stride 1: plain GEMM
    (2, 256, 512, 14, 14, 1, 1, 2, 0, None),   # strided 1x1 downsample
    (2, 128, 128, 15, 15, 3, 3, 2, 1, "relu"), # strided 3x3
    (1, 3, 64, 32, 32, 7, 7, 2, 3, "relu"),    # 3-channel stem: space-to-depth or element-wise gather
    (3, 24, 40, 9, 11, 3, 3, 1, 1, None),      # ragged M, N < 64
    (1, 12, 20, 7, 7, 3, 3, 1, 1, "relu"),     # C_IN % 8 != 0
    (1, 512, 2048, 7, 7, 1, 1, 1, 0, None),    # deep 1x1 (M = 49)
    (2, 64, 96, 10, 10, 3, 3, 1, 0, None),     # N = 96: BN=128 tile, half-empty
    (2, 512, 512, 6, 6, 3, 3, 1, 1, "relu"),   # deep 3x3 on a small grid: split-K
    (2, 256, 256, 14, 14, 3, 3, 1, 1, "relu"), # ResNet stage 3 shape: the band-tiled kernel
    (1, 20, 48, 8, 8, 5, 5, 1, 2, None),       # element-wise gather, 5x5
    (2, 3, 32, 29, 31, 7, 7, 2, 3, None),      # stride-2 space-to-depth, odd sizes
    (1, 3, 16, 20, 20, 3, 3, 2, 1, "relu"),    # space-to-depth, 3x3 -> 2x2
    (1, 1, 8, 15, 15, 5, 5, 2, 2, None),       # space-to-depth, one channel
    (2, 6, 24, 12, 12, 4, 4, 2, 0, "relu"),    # space-to-depth, C2 = 24, even kernel
]


# cases whose fastest plan needs stream scratch (split-K partials or the
# space-to-depth copy) on a 256-CU device
SCRATCH_CASES = {BF16_CASES[i] for i in (4, 9, 12, 13, 14, 15)}


@pytest.mark.parametrize("case", BF16_CASES)
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_bf16_nhwc_mfma(dev, orc, case, with_bias, scratch):
    B, Cin, Cout, H, W, KH, KW, s, p, act = case
    print(f"[conv bf16] {case} bias={with_bias} scratch={scratch}", flush=True)
    rng = np.random.default_rng(Cin * 7 + Cout + H)
    x = rb(rng.standard_normal((B, H, W, Cin), dtype=np.float32))
    w = rb((rng.standard_normal((Cout, KH, KW, Cin), dtype=np.float32) * np.sqrt(2.0 / (Cin * KH * KW))).astype(np.float32))
    b = rb(rng.normal(0, 0.1, Cout).astype(np.float32)) if with_bias else None
    need = K.conv2d_workspace_size((B, H, W, Cin), (Cout, KH, KW, Cin), s, p, 1, tg.bf16, "nhwc")
    if dev.info()["compute_units"] == 256:
        assert (need > 0) == (case in SCRATCH_CASES), need
    if scratch == "workspace" and need == 0:
        pytest.skip("no scratch plan at this shape: same path as scratch=none")

    def run():
        return K.conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16),
                        dev.upload(to_bf16(b), tg.bf16) if with_bias else None, s, p, 1, act,
                        layout="nhwc").to_host()

    if scratch == "workspace":
        with stream_workspace(dev, need):
            got = run()
    else:
        got = run()
    ref = orc.conv2d_nhwc(x, w, b, stride=s, padding=p)
    if act == "relu":
        ref = orc.relu(ref)
    check_bf16(got, ref, str(case))


def test_bf16_nhwc_large_tile(dev, orc):
    # batch 64, 56x56, 64 -> 256, 3x3: M = 200704 fills the chip with 256 x 256
    # tiles (large-tile implicit-GEMM kernel); images 0 and 63 vs the oracle
    B, H, Cin, Cout = 64, 56, 64, 256
    rng = np.random.default_rng(56)
    x = rb(rng.standard_normal((B, H, H, Cin), dtype=np.float32))
    w = rb((rng.standard_normal((Cout, 3, 3, Cin), dtype=np.float32) * np.sqrt(2.0 / (Cin * 9))).astype(np.float32))
    b = rb(rng.normal(0, 0.1, Cout).astype(np.float32))
    print("[conv bf16 large tile] B=64 56x56 64->256 3x3", flush=True)
    got = K.conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16),
                   dev.upload(to_bf16(b), tg.bf16), 1, 1, 1, "relu", layout="nhwc").to_host()
    for i in (0, B - 1):
        ref = orc.relu(orc.conv2d_nhwc(x[i:i + 1], w, b, stride=1, padding=1))
        check_bf16(got[i:i + 1], ref, f"image {i}")


@pytest.mark.parametrize("act,bn", [("gelu", False), ("silu", True), (None, False)])
def test_bf16_nhwc_persistent_strided_1x1(dev, orc, act, bn):
    # batch 42, 56x56, 256 -> 512, 1x1 stride 2 (a ResNet downsample at a
    # ragged batch): M = 32928 rows, 1032 tiles of 128 x 128, K = 256 -> the
    # persistent kernel on the strided gather; with bn the folded BatchNorm's
    # scale and shift are its epilogue coefficients.  One output pixel of
    # every 128-row tile, and images 0 and 41 whole, vs the oracle.
    B, H, Cin, Cout = 42, 56, 256, 512
    print(f"[conv bf16 persistent] B=42 56x56 256->512 1x1/2 act={act} bn={bn}", flush=True)
    rng = np.random.default_rng(4256)
    xb = to_bf16(rng.random((B, H, H, Cin), dtype=np.float32))
    wb = to_bf16((rng.standard_normal((Cout, 1, 1, Cin), dtype=np.float32) * np.sqrt(2.0 / Cin)).astype(np.float32))
    x, w = from_bf16(xb), from_bf16(wb)
    assert K.conv2d_workspace_size((B, H, H, Cin), (Cout, 1, 1, Cin), 2, 0, 1, tg.bf16, "nhwc") == 0
    if bn:
        scale = rng.uniform(0.5, 1.5, Cout).astype(np.float32)
        shift = rng.normal(0, 0.1, Cout).astype(np.float32)
        got = K.conv2d_bn_act(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(scale), dev.upload(shift),
                              2, 0, 1, act, layout="nhwc").to_host()
        bias = None
    else:
        bias = rb(rng.normal(0, 0.1, Cout).astype(np.float32))
        got = K.conv2d(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(to_bf16(bias), tg.bf16),
                       2, 0, 1, act, layout="nhwc").to_host()

    def post(ref):
        if bn:
            ref = ref * scale + shift
        return ref if act is None else {"silu": orc.silu, "gelu": orc.gelu}[act](ref)

    m = B * 28 * 28
    starts = np.arange(0, m, 128)
    pix = starts + (rng.random(starts.size) * np.minimum(128, m - starts)).astype(np.int64)
    assert np.all(np.isfinite(from_bf16(got)))
    check_bf16(got.reshape(m, Cout)[pix], post(orc.conv2d_nhwc_pixels(x, w, pix, bias, stride=2, padding=0)),
               f"{pix.size} sampled pixels")
    for i in (0, B - 1):
        check_bf16(got[i:i + 1], post(orc.conv2d_nhwc(x[i:i + 1], w, bias, stride=2, padding=0)), f"image {i}")


BAND_CASES = [
    # B, H, W, Cin, Cout, K, stride, pad, act, bias/bn: shapes the row-band
    # kernel takes (weights resident in LDS, input row bands with their halo
    # staged once per channel chunk)
    (3, 56, 56, 64, 64, 3, 1, 1, "relu", "bias"),    # the 56x56 ResNet 3x3 at a ragged batch
    (2, 58, 58, 64, 64, 3, 1, 0, "gelu", "bias"),    # no padding: a 58-wide input for 56 outputs
    (2, 56, 56, 64, 64, 3, 1, 1, "silu", "bn"),      # folded BatchNorm scale / shift
    (1, 56, 56, 64, 64, 3, 1, 1, None, None),        # no bias
    (2, 224, 224, 3, 64, 7, 2, 3, "relu", "bias"),   # the stem: raw rows, space-to-depth formed in LDS
    (1, 224, 224, 3, 64, 7, 2, 3, "gelu", "bn"),
    (3, 100, 224, 3, 64, 7, 2, 3, "silu", "bias"),   # the raw stem on a short image (OH 50)
    (2, 101, 224, 3, 64, 7, 2, 3, "relu", "bias"),   # odd OH: the space-to-depth pass + band kernel
    (1, 64, 96, 3, 64, 7, 2, 3, None, "bias"),       # another width: the space-to-depth pass
]


@pytest.mark.parametrize("case", BAND_CASES)
def test_bf16_nhwc_band(dev, orc, case):
    B, H, W, Cin, Cout, k, s, p, act, post = case
    print(f"[conv bf16 band] {case}", flush=True)
    rng = np.random.default_rng(H + 7 * W + Cin + k + (0 if act is None else len(act)))
    xb = to_bf16(rng.random((B, H, W, Cin), dtype=np.float32))
    wb = to_bf16((rng.standard_normal((Cout, k, k, Cin), dtype=np.float32) * np.sqrt(2.0 / (Cin * k * k))).astype(np.float32))
    x, w = from_bf16(xb), from_bf16(wb)
    oh, ow = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    need = K.conv2d_workspace_size((B, H, W, Cin), (Cout, k, k, Cin), s, p, 1, tg.bf16, "nhwc")
    bias = scale = shift = None
    with stream_workspace(dev, need):
        if post == "bn":
            scale = rng.uniform(0.5, 1.5, Cout).astype(np.float32)
            shift = rng.normal(0, 0.1, Cout).astype(np.float32)
            got = K.conv2d_bn_act(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(scale),
                                  dev.upload(shift), s, p, 1, act, layout="nhwc").to_host()
        else:
            if post == "bias":
                bias = rb(rng.normal(0, 0.1, Cout).astype(np.float32))
            got = K.conv2d(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16),
                           dev.upload(to_bf16(bias), tg.bf16) if bias is not None else None, s, p, 1, act,
                           layout="nhwc").to_host()
        dev.synchronize()

    def finish(ref):
        if post == "bn":
            ref = ref * scale + shift
        return ref if act is None else {"relu": orc.relu, "silu": orc.silu, "gelu": orc.gelu}[act](ref)

    assert got.shape == (B, oh, ow, Cout)
    check_bf16(got, finish(orc.conv2d_nhwc(x, w, bias, stride=s, padding=p)), "all images")
    if Cin == 3 and W == 224 and oh % 2 == 0:
        assert need == 0, need  # the raw stem needs no space-to-depth scratch


TILE_CASES = [
    # B, H, W, Cin, Cout, pad, act, post, int8: stride-1 bf16 3x3 convs with
    # 14- and 28-wide outputs take the band-tiled kernel (a band of 196 output
    # pixels x 64 channels per workgroup, input rows with their halo and the
    # chunk's weights staged per 32 input channels), 7x7 outputs a band of
    # two images; the int8 cases run the implicit GEMM
    (5, 14, 14, 256, 256, 1, "relu", "bias", False),   # the 14x14 ResNet 3x3 at a ragged batch
    (2, 14, 14, 64, 128, 1, "gelu", "bn", False),      # two channel tiles, folded BatchNorm
    (2, 16, 16, 96, 64, 0, None, None, False),         # no padding: 16 -> 14, three chunks
    # more units than workgroups (one per CU): workgroups walk several bands,
    # with one chunk per band (every stage ends a band, and the channel tile
    # changes between a workgroup's bands) or two
    (90, 14, 14, 32, 192, 1, "silu", None, False),
    (140, 14, 14, 64, 128, 1, "relu", "bias", False),
    (3, 28, 28, 128, 128, 1, "relu", "bias", False),   # the 28x28 ResNet 3x3
    (1, 28, 28, 32, 192, 1, "silu", None, False),      # one chunk, three channel tiles
    (30, 28, 28, 64, 192, 1, "relu", None, False),     # 360 bands x tiles: two per workgroup
    # 7x7 outputs: two whole images per band (the last band of an odd batch
    # half empty)
    (5, 7, 7, 64, 128, 1, "relu", "bias", False),
    (4, 7, 7, 96, 64, 1, None, "bn", False),           # three chunks
    (600, 7, 7, 32, 64, 1, "silu", None, False),       # 300 bands: several per workgroup
    (3, 9, 9, 64, 64, 0, "gelu", "bias", False),       # no padding: 9 -> 7
    (3, 28, 28, 256, 256, 1, None, "bias", True),      # the W8A16 conv at a ragged batch
    (2, 28, 28, 64, 128, 1, "relu", None, True),
]


S2_TILE_CASES = [
    # B, H, W, Cin, Cout, pad, act, post, int8: stride-2 bf16 3x3 convs with
    # 7x7 and 14x14 outputs take the band-tiled kernel in its stride-2 mode
    # (two images or half an image per band, the halo's columns as even and
    # odd phase planes, two waves per pixel block); 28-wide outputs run the
    # implicit GEMM
    (5, 14, 14, 512, 512, 1, "relu", "bias", False),   # the 7x7 ResNet stride-2 3x3, ragged batch
    (3, 13, 13, 64, 128, 1, None, "bn", False),        # odd input: the last column and row are padding
    (2, 15, 15, 32, 64, 0, "silu", None, False),       # no padding: 15 -> 7
    (600, 14, 14, 32, 64, 1, "silu", None, False),     # 300 bands: several per workgroup
    (3, 28, 28, 256, 256, 1, "relu", "bias", False),   # the 14x14 ResNet stride-2 3x3
    (2, 27, 27, 64, 64, 1, "gelu", None, False),
    (40, 28, 28, 64, 192, 1, "relu", None, False),     # 240 units, three channel tiles
    (2, 56, 56, 128, 128, 1, "relu", "bias", False),   # the 28x28 ResNet stride-2 3x3
    (20, 56, 56, 64, 128, 1, None, "bn", False),       # 280 units
    (2, 28, 28, 256, 256, 1, None, "bias", True),      # int8 weights: the implicit GEMM (no workspace)
]


@pytest.mark.parametrize("case", TILE_CASES)
def test_nhwc_band_tiles(dev, orc, case):
    run_band_tile_case(dev, orc, case, 1)


@pytest.mark.parametrize("case", S2_TILE_CASES)
def test_nhwc_band_tiles_stride2(dev, orc, case):
    run_band_tile_case(dev, orc, case, 2)


def run_band_tile_case(dev, orc, case, st):
    B, H, W, Cin, Cout, p, act, post, int8 = case
    print(f"[conv band tiles] stride {st} {case}", flush=True)
    rng = np.random.default_rng(H * W + Cin + Cout + p)
    xb = to_bf16(rng.standard_normal((B, H, W, Cin), dtype=np.float32))
    x = from_bf16(xb)
    oh, ow = (H + 2 * p - 3) // st + 1, (W + 2 * p - 3) // st + 1
    bias = scale = shift = None
    if int8:
        q, qs = quantized_conv_weight(orc, rng, Cout, 3, 3, Cin)
        w = orc.dequantize_affine(q.reshape(-1), qs, None, q.shape, "channel", 0)
        if post == "bias":
            bias = rng.normal(0, 0.1, Cout).astype(np.float32)
        got = K.w8a16_conv2d(dev.upload(xb, tg.bf16), dev.upload(q), dev.upload(qs),
                             dev.upload(bias) if bias is not None else None, st, p, act=act).to_host()
    else:
        wb = to_bf16((rng.standard_normal((Cout, 3, 3, Cin), dtype=np.float32) * np.sqrt(2.0 / (9 * Cin))).astype(np.float32))
        w = from_bf16(wb)
        if post == "bn":
            scale = rng.uniform(0.5, 1.5, Cout).astype(np.float32)
            shift = rng.normal(0, 0.1, Cout).astype(np.float32)
            got = K.conv2d_bn_act(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(scale),
                                  dev.upload(shift), st, p, 1, act, layout="nhwc").to_host()
        else:
            if post == "bias":
                bias = rb(rng.normal(0, 0.1, Cout).astype(np.float32))
            got = K.conv2d(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16),
                           dev.upload(to_bf16(bias), tg.bf16) if bias is not None else None, st, p, 1, act,
                           layout="nhwc").to_host()

    def finish(ref):
        if post == "bn":
            ref = ref * scale + shift
        return ref if act is None else {"relu": orc.relu, "silu": orc.silu, "gelu": orc.gelu}[act](ref)

    assert got.shape == (B, oh, ow, Cout)
    assert np.all(np.isfinite(from_bf16(got)))
    check_bf16(got, finish(orc.conv2d_nhwc(x, w, bias, stride=st, padding=p)), f"stride {st} {case}")


STREAM_CASES = [
    # B, H, W, Cin, Cout, act: 1x1 stride-1 convs with M = B*H*W >= 16384 and
    # C_IN, C_OUT in {64, 128, 256} take the streaming kernel
    (8, 48, 48, 64, 256, "relu"),    # M = 18432 (whole 32-row blocks)
    (7, 50, 50, 256, 64, None),      # M = 17500: last block has 28 rows
    (9, 45, 45, 64, 128, "silu"),    # M = 18225: ragged, SiLU epilogue
    (5, 61, 61, 128, 128, "gelu"),   # M = 18605: ragged, GELU epilogue
    (4, 64, 64, 256, 128, "relu"),   # M = 16384: the smallest streamed M
]


@pytest.mark.parametrize("case", STREAM_CASES)
@pytest.mark.parametrize("with_bias", [True, False])
def test_bf16_nhwc_stream_1x1(dev, orc, case, with_bias):
    B, H, W, Cin, Cout, act = case
    print(f"[conv bf16 stream 1x1] {case} bias={with_bias}", flush=True)
    rng = np.random.default_rng(Cin + 3 * Cout + H)
    x = rb(rng.standard_normal((B, H, W, Cin), dtype=np.float32))
    w = rb((rng.standard_normal((Cout, 1, 1, Cin), dtype=np.float32) * np.sqrt(2.0 / Cin)).astype(np.float32))
    b = rb(rng.normal(0, 0.1, Cout).astype(np.float32)) if with_bias else None
    assert K.conv2d_workspace_size((B, H, W, Cin), (Cout, 1, 1, Cin), 1, 0, 1, tg.bf16, "nhwc") == 0
    got = K.conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16),
                   dev.upload(to_bf16(b), tg.bf16) if with_bias else None, 1, 0, 1, act, layout="nhwc").to_host()
    ref = orc.conv2d_nhwc(x, w, b, stride=1, padding=0)
    if act is not None:
        ref = {"relu": orc.relu, "silu": orc.silu, "gelu": orc.gelu}[act](ref)
    check_bf16(got, ref, str(case))


def test_bf16_nchw_and_grouped_direct(dev, orc):
    rng = np.random.default_rng(5)
    x = rb(rng.standard_normal((2, 8, 10, 10), dtype=np.float32))
    w = rb(rng.normal(0, 0.3, (8, 4, 3, 3)).astype(np.float32))
    got = K.conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(to_bf16(w), tg.bf16), None, 1, 1, 2).to_host()
    check_bf16(got, orc.conv2d_nchw(x, w, None, padding=1, groups=2), "bf16 nchw grouped")
    xh = np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    wh = np.ascontiguousarray(w.transpose(0, 2, 3, 1))
    got = K.conv2d(dev.upload(to_bf16(xh), tg.bf16), dev.upload(to_bf16(wh), tg.bf16), None, 1, 1, 2,
                   layout="nhwc").to_host()
    check_bf16(got, orc.conv2d_nhwc(xh, wh, None, padding=1, groups=2), "bf16 nhwc grouped")


def quantized_conv_weight(orc, rng, cout, kh, kw, cin):
    wf = rng.normal(0, 0.02, (cout, kh, kw, cin)).astype(np.float32)
    q, s, z, _ = orc.quantize_affine(wf, wf.shape, "channel", 0)
    return q.reshape(wf.shape), s


@pytest.mark.parametrize("B,Cin,Cout,H,act", [(2, 256, 256, 28, None), (1, 64, 96, 9, "relu"),
                                              (1, 24, 16, 8, None), (3, 32, 48, 14, "relu")])
@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_w8a16_conv(dev, orc, B, Cin, Cout, H, act, scratch):
    # int8 3x3 conv (the W8A16 conv workload at reduced batch; Cin=24 takes the
    # fallback kernel); given a workspace, the first case splits along K
    print(f"[w8a16 conv] B={B} Cin={Cin} Cout={Cout} H={H} scratch={scratch}", flush=True)
    rng = np.random.default_rng(Cin + H)
    x = rb(rng.standard_normal((B, H, H, Cin), dtype=np.float32))
    q, s = quantized_conv_weight(orc, rng, Cout, 3, 3, Cin)
    bias = rng.normal(0, 0.1, Cout).astype(np.float32)
    need = K.conv2d_workspace_size((B, H, H, Cin), (Cout, 3, 3, Cin), 1, 1, 1, tg.i8)
    if scratch == "workspace" and need == 0:
        pytest.skip("no scratch plan at this shape: same path as scratch=none")

    def run():
        return K.w8a16_conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(q), dev.upload(s),
                              dev.upload(bias), 1, 1, act=act).to_host()

    if scratch == "workspace":
        with stream_workspace(dev, need):
            got = run()
    else:
        got = run()
    wdeq = orc.dequantize_affine(q.reshape(-1), s, None, q.shape, "channel", 0)
    ref = orc.conv2d_nhwc(x, wdeq, bias, stride=1, padding=1)
    if act == "relu":
        ref = orc.relu(ref)
    check_bf16(got, ref, "w8a16 conv")


@pytest.mark.parametrize("scratch", ["none", "workspace"])
def test_w8a16_conv_config_batch32(dev, orc, scratch):
    # 32 x 256 x 28 x 28, 3x3 p1: the whole output against the oracle; without
    # scratch the int8 implicit GEMM, with it the band-tiled kernel on a bf16
    # copy of the weights
    B, C, H = 32, 256, 28
    rng = np.random.default_rng(0x7EE70004)
    x = rb(rng.standard_normal((B, H, H, C), dtype=np.float32))
    q, s = quantized_conv_weight(orc, rng, C, 3, 3, C)
    need = K.conv2d_workspace_size((B, H, H, C), (C, 3, 3, C), 1, 1, 1, tg.i8)
    assert need == C * 9 * C * 2, need
    print(f"[w8a16 conv config] 32x256x28x28 scratch={scratch}", flush=True)

    def run():
        return K.w8a16_conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(q), dev.upload(s), None, 1, 1).to_host()

    if scratch == "workspace":
        with stream_workspace(dev, need):
            got = run()
    else:
        got = run()
    assert np.all(np.isfinite(from_bf16(got)))
    wdeq = orc.dequantize_affine(q.reshape(-1), s, None, q.shape, "channel", 0)
    ref = orc.conv2d_nhwc(x, wdeq, None, stride=1, padding=1)
    check_bf16(got, ref, "all 32 images")


@pytest.mark.parametrize("scratch", ["none", "short", "workspace"])
def test_w8a16_conv_large_tile(dev, orc, scratch):
    # 128 x 256 x 28 x 28, 3x3 p1, with bias and ReLU: M = 100352 gives 392
    # 256 x 256 tiles, so without scratch (or with less than the bf16 weight
    # copy needs) the implicit GEMM takes the large-tile LDS-DMA kernel on int8
    # weights converted in registers; with the reported workspace the
    # band-tiled kernel runs on the bf16 copy; images 0, 77 and 127 against
    # the oracle
    B, C, H = 128, 256, 28
    rng = np.random.default_rng(0x7EE70128)
    x = rb(rng.standard_normal((B, H, H, C), dtype=np.float32))
    q, s = quantized_conv_weight(orc, rng, C, 3, 3, C)
    bias = rng.normal(0, 0.1, C).astype(np.float32)
    need = K.conv2d_workspace_size((B, H, H, C), (C, 3, 3, C), 1, 1, 1, tg.i8)
    assert need == C * 9 * C * 2, need
    print(f"[w8a16 conv large tile] 128x256x28x28 scratch={scratch}", flush=True)

    def run():
        return K.w8a16_conv2d(dev.upload(to_bf16(x), tg.bf16), dev.upload(q), dev.upload(s), dev.upload(bias), 1, 1,
                              act="relu").to_host()

    if scratch == "none":
        got = run()
    else:
        with stream_workspace(dev, need if scratch == "workspace" else need - 16):
            got = run()
    wdeq = orc.dequantize_affine(q.reshape(-1), s, None, q.shape, "channel", 0)
    for b in (0, 77, B - 1):
        ref = orc.relu(orc.conv2d_nhwc(x[b:b + 1], wdeq, bias, stride=1, padding=1))
        check_bf16(got[b:b + 1], ref, f"image {b}")


GROUPED_CASES = [
    # B, H, W, Cin, Cout, K, stride, pad, groups, act, post: bf16 NHWC grouped
    # convs with >= 16 output channels per group run all groups in one
    # implicit-GEMM launch (input channels of group g at a pixel stride of
    # C_IN); fewer per group stay on the direct kernel
    (2, 14, 14, 64, 128, 3, 1, 1, 4, "relu", "bias"),   # 16 -> 32 per group
    (3, 9, 11, 128, 128, 3, 2, 1, 8, None, None),       # strided, 16 -> 16
    (2, 10, 10, 32, 64, 1, 1, 0, 2, "silu", "bias"),    # 1x1: plain rows at a C_IN row stride
    (2, 12, 12, 24, 48, 3, 1, 1, 2, None, "bn"),        # 12 channels per group: element gather
    (4, 7, 7, 256, 512, 3, 1, 1, 2, "gelu", "bias"),    # deep K per group (1152)
    (1, 8, 8, 64, 64, 3, 1, 1, 8, None, None),          # 8 -> 8 per group: the direct kernel
]


@pytest.mark.parametrize("case", GROUPED_CASES)
def test_bf16_nhwc_grouped(dev, orc, case):
    B, H, W, cin, cout, k, s, p, G, act, post = case
    print(f"[conv grouped] {case}", flush=True)
    rng = np.random.default_rng(cin * 7 + cout + G)
    xb = to_bf16(rng.standard_normal((B, H, W, cin), dtype=np.float32))
    wb = to_bf16((rng.standard_normal((cout, k, k, cin // G), dtype=np.float32) *
                  np.float32(np.sqrt(2.0 / (k * k * cin // G)))))
    x, w = from_bf16(xb), from_bf16(wb)
    bias = scale = shift = None
    if post == "bn":
        scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
        shift = rng.normal(0, 0.1, cout).astype(np.float32)
        got = K.conv2d_bn_act(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(scale),
                              dev.upload(shift), s, p, G, act, layout="nhwc").to_host()
    else:
        if post == "bias":
            bias = from_bf16(to_bf16(rng.normal(0, 0.1, cout).astype(np.float32)))
        got = K.conv2d(dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16),
                       dev.upload(to_bf16(bias), tg.bf16) if bias is not None else None, s, p, G, act,
                       layout="nhwc").to_host()
    ref = orc.conv2d_nhwc(x, w, bias, stride=s, padding=p, groups=G)
    if post == "bn":
        ref = ref * scale + shift
    if act is not None:
        ref = {"relu": orc.relu, "silu": orc.silu, "gelu": orc.gelu}[act](ref)
    check_bf16(got, ref, str(case))
