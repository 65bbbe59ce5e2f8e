"""GPU: compressed-tensors int8 checkpoints feeding the W8A16 kernels.

Files in teeny-quant's convention (utilities/teeny-quant/src/format.rs:16-35:
foo.weight I8, foo.weight_scale F32, foo.weight_zero_point I32 when
asymmetric, quantization_config in the header) are written with the oracle
as the quantizer, loaded by the native reader straight into device buffers
and run through w8a16_linear / w8a16_conv2d; the results are checked against
the oracle's dequantize_affine + linear / conv.  The library's own GPU writer
(quantize_checkpoint) must produce the same quantized tensors bit for bit,
and dequantize() of any int8 scheme must equal dequantize_affine
(format.rs:249-289, affine.rs:151-161) exactly."""
import numpy as np
import pytest

import teenygrad_amd as tg
from gpu_util import check_bf16
from teenygrad_amd import kernels as K
from teenygrad_amd.checkpoint import Checkpoint, quantize_checkpoint
from teenygrad_amd.dtypes import from_bf16, to_bf16
from test_checkpoint import oracle_ct_file

pytestmark = pytest.mark.gpu


def rb(a):
    return from_bf16(to_bf16(a))


@pytest.mark.parametrize("gran", ["channel", "tensor"])
def test_checkpoint_to_w8a16_linear(dev, orc, tmp_path, gran):
    rng = np.random.default_rng(3)
    m, k, n = 300, 512, 384
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    blob, _ = oracle_ct_file(orc, {"layers.0.mlp.weight": w, "layers.0.mlp.bias": bias}, gran, 0)
    path = tmp_path / "model.safetensors"
    path.write_bytes(blob)
    x = rb(rng.standard_normal((m, k), dtype=np.float32))
    print(f"[checkpoint] w8a16 linear from a {gran} file", flush=True)
    with Checkpoint(str(path)) as ck:
        q, s = ck.load_w8a16("layers.0.mlp.weight")
        b = ck.to_device("layers.0.mlp.bias", tg.f32)
    assert q.shape == (n, k) and s.shape == (n,)
    y = K.w8a16_linear(dev.upload(to_bf16(x), tg.bf16), q, s, b).to_host()
    oq, os_, _, _ = orc.quantize_affine(w, [n, k], gran, 0)
    wdeq = orc.dequantize_affine(oq, os_, None, [n, k], gran, 0)
    check_bf16(y, orc.linear(x, wdeq, bias), f"w8a16 from checkpoint ({gran})")
    if gran == "tensor":
        np.testing.assert_array_equal(s.to_host(), np.full(n, os_[0], np.float32))


@pytest.mark.parametrize("kh,kw", [(3, 3), (1, 3)])
def test_checkpoint_to_w8a16_conv(dev, orc, tmp_path, kh, kw):
    # teeny-quant stores a conv weight in the reference's order [C_OUT, C_IN,
    # KH, KW] (conv2d.rs:43-156); the loader repacks it for the NHWC conv.
    # A non-square kernel makes a swapped KH/KW visible too.
    rng = np.random.default_rng(4)
    B, H, cin, cout = 2, 14, 64, 128
    w = rng.normal(0, 0.02, (cout, cin, kh, kw)).astype(np.float32)
    blob, _ = oracle_ct_file(orc, {"conv.weight": w}, "channel", 0)
    (tmp_path / "c.safetensors").write_bytes(blob)
    x = rb(rng.standard_normal((B, H, H, cin), dtype=np.float32))
    print(f"[checkpoint] w8a16 conv {kh}x{kw} from an NCHW-ordered file", flush=True)
    with Checkpoint(str(tmp_path / "c.safetensors")) as ck:
        q, s = ck.load_w8a16("conv.weight")
    assert q.shape == (cout, kh, kw, cin)
    ph, pw = kh // 2, kw // 2
    y = K.w8a16_conv2d(dev.upload(to_bf16(x), tg.bf16), q, s, None, 1, (ph, pw)).to_host()
    oq, os_, _, _ = orc.quantize_affine(w, list(w.shape), "channel", 0)
    wdeq = orc.dequantize_affine(oq, os_, None, list(w.shape), "channel", 0).reshape(w.shape)
    ref = orc.conv2d_nchw(np.ascontiguousarray(x.transpose(0, 3, 1, 2)), wdeq, None, stride=1,
                          padding=(ph, pw)).transpose(0, 2, 3, 1)
    check_bf16(y, ref, "w8a16 conv from checkpoint")
    # the repacked int8 weights are exactly the file's, transposed
    np.testing.assert_array_equal(q.to_host().reshape(cout, kh, kw, cin),
                                  oq.reshape(cout, cin, kh, kw).transpose(0, 2, 3, 1))


@pytest.mark.parametrize("gran,axis,gs,sym", [("channel", 0, 1, True), ("group", 1, 32, True),
                                              ("channel", 1, 1, False), ("tensor", 0, 1, False)])
def test_gpu_writer_matches_oracle_and_dequantizes(dev, orc, gran, axis, gs, sym):
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.03, (48, 96)).astype(np.float32)
    w.reshape(-1)[::7] *= 4.0
    bias = rng.normal(0, 0.1, 48).astype(np.float32)
    tensors = {"fc.weight": w, "fc.bias": bias}
    ours = quantize_checkpoint(tensors, gran, axis, gs, sym)
    ref, parts = oracle_ct_file(orc, tensors, gran, axis, gs, sym)
    with Checkpoint(image=ours) as a, Checkpoint(image=ref) as b:
        assert a.tensors().keys() == b.tensors().keys()
        for name in b.tensors():
            np.testing.assert_array_equal(a.read(name), b.read(name), err_msg=name)
        assert a.quant_scheme() == b.quant_scheme()
        d = a.dequantize("fc.weight").to_host()
        oq, os_, oz, _ = orc.quantize_affine(w, list(w.shape), gran, axis, gs, sym)
        np.testing.assert_array_equal(d, orc.dequantize_affine(oq, os_, None if sym else oz, list(w.shape), gran,
                                                               axis, gs))
