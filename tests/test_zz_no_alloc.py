"""GPU: teeny_conv2d_bias_forward_noalloc, the conv entry point that allocates
nothing and takes its scratch from a fixed device array inside the library.

Called through the C ABI and compared with teeny_conv2d_bias_forward given a
stream workspace (the same plan and kernels, so the outputs are bit-identical)
and with the oracle on sampled output pixels, for the two scratch users: the
split-K partial sums of a deep 3x3 conv on a small grid, and the
space-to-depth copy of a 3-channel stride-2 7x7 conv (the 224-wide RGB stem
itself forms that copy in LDS and needs no scratch).  Each runs twice in a
row, the second call on a smaller input, so the second reads none of the
first call's leftovers."""
import ctypes

import numpy as np
import pytest

import teenygrad_amd as tg
from gpu_util import check_bf16, stream_workspace
from teenygrad_amd import _lib
from teenygrad_amd import kernels as K
from teenygrad_amd._lib import check, lib
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu

# (B, C_IN, C_OUT, H, K, stride, pad): first the larger input, then the smaller
SPLIT_K = [(64, 512, 512, 6, 3, 1, 1), (2, 512, 512, 6, 3, 1, 1)]
S2D = [(16, 3, 64, 160, 7, 2, 3), (3, 3, 64, 61, 7, 2, 3)]


def make(shape, seed):
    B, cin, cout, h, k, s, p = shape
    rng = np.random.default_rng(seed)
    x = to_bf16(rng.random((B, h, h, cin), dtype=np.float32))
    w = to_bf16((rng.standard_normal((cout, k, k, cin), dtype=np.float32) * np.float32(np.sqrt(2.0 / (cin * k * k)))))
    b = to_bf16(rng.normal(0, 0.01, cout).astype(np.float32))
    return x, w, b


def conv_call(fn, xd, wd, bd, yd, shape):
    B, cin, cout, h, k, s, p = shape
    oh = (h + 2 * p - k) // s + 1
    prm = _lib.Conv2dParams(k, k, s, s, p, p, 1, _lib.ACT_RELU)
    check(fn(xd.ptr, wd.ptr, bd.ptr, yd.ptr, B, cin, cout, h, h, oh, oh, ctypes.byref(prm), _lib.BF16,
             _lib.NHWC, None))


@pytest.mark.parametrize("pair", [SPLIT_K, S2D], ids=["split_k", "space_to_depth"])
def test_noalloc_matches_workspace_entry(dev, orc, pair):
    for i, shape in enumerate(pair):
        B, cin, cout, h, k, s, p = shape
        oh = (h + 2 * p - k) // s + 1
        need = K.conv2d_workspace_size((B, h, h, cin), (cout, k, k, cin), s, p, 1, tg.bf16, "nhwc")
        print(f"[noalloc] call {i + 1}: {shape} scratch need {need} B", flush=True)
        assert 0 < need <= 32 << 20
        x, w, b = make(shape, 100 + i)
        xd, wd, bd = dev.upload(x, tg.bf16), dev.upload(w, tg.bf16), dev.upload(b, tg.bf16)
        y_static = tg.Buffer(tg.bf16, (B, oh, oh, cout))
        y_ws = tg.Buffer(tg.bf16, (B, oh, oh, cout))
        conv_call(lib.teeny_conv2d_bias_forward_noalloc, xd, wd, bd, y_static, shape)
        dev.synchronize()
        with stream_workspace(dev, need):
            conv_call(lib.teeny_conv2d_bias_forward, xd, wd, bd, y_ws, shape)
        got, want = y_static.to_host(), y_ws.to_host()
        np.testing.assert_array_equal(got, want)
        # and against the oracle on one output pixel per 128-row tile
        m = B * oh * oh
        pix = np.arange(0, m, 128) + (np.arange(-(-m // 128)) * 37) % np.minimum(128, m - np.arange(0, m, 128))
        ref = orc.relu(orc.conv2d_nhwc_pixels(from_bf16(x), from_bf16(w), pix, from_bf16(b), stride=s, padding=p))
        check_bf16(got.reshape(m, cout)[pix], ref, f"call {i + 1} {shape}")


def test_raw_stem_needs_no_scratch():
    # the 224-wide stem reads the raw image and forms the space-to-depth
    # input in LDS: no workspace, so the no-allocation entry takes it too
    assert K.conv2d_workspace_size((64, 224, 224, 3), (64, 7, 7, 3), 2, 3, 1, tg.bf16, "nhwc") == 0
