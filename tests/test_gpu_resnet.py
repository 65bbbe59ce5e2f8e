"""GPU parity: the 53 convolutions of ResNet-50 at batch 64, 224x224 input,
bf16 NHWC with BN folded into a bias and ReLU fused where the network has it
(the ResNet-50 conv stack workload), each at its own shape and tile plan,
with and without the stream workspace the benchmark attaches.

Per layer, the whole output (all 64 images, every pixel and channel) is
checked against the oracle, for each scratch mode.
Reference semantics: conv2d_bias_forward, kernels/teeny-kernels/src/nn/conv/
conv2d.rs:642-764 (NCHW there; NHWC here, an exact transpose)."""
import numpy as np
import pytest

import teenygrad_amd as tg
from gpu_util import check_bf16, stream_workspace
from teenygrad_amd import kernels as K
from teenygrad_amd import synthetic
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu

BATCH = 64
LAYERS = synthetic.resnet50_convs()


@pytest.mark.parametrize("layer", LAYERS, ids=[l[0] for l in LAYERS])
def test_resnet50_layer_batch64(dev, orc, layer):
    name, cin, cout, h, k, s, p, relu = layer
    oh = (h + 2 * p - k) // s + 1
    print(f"[resnet50 b64] {name}: {cin}->{cout} {h}x{h} k{k} s{s} p{p} relu={relu}", flush=True)
    rng = np.random.default_rng(synthetic.workload_seed(4, LAYERS.index(layer)))
    xb = to_bf16(rng.random((BATCH, h, h, cin), dtype=np.float32))
    wb = to_bf16((rng.standard_normal((cout, k, k, cin), dtype=np.float32)
                  * np.float32(np.sqrt(2.0 / (cin * k * k)))).astype(np.float32))
    bb = to_bf16(rng.normal(0, 0.01, cout).astype(np.float32))
    x, w, b = from_bf16(xb), from_bf16(wb), from_bf16(bb)
    xd, wd, bd = dev.upload(xb, tg.bf16), dev.upload(wb, tg.bf16), dev.upload(bb, tg.bf16)
    act = "relu" if relu else None
    need = K.conv2d_workspace_size((BATCH, h, h, cin), (cout, k, k, cin), s, p, 1, tg.bf16, "nhwc")

    def run():
        return K.conv2d(xd, wd, bd, s, p, 1, act, "nhwc").to_host()

    outs = {"none": run()}
    if need > 0:
        with stream_workspace(dev, need):
            outs["workspace"] = run()
    del xd

    ref = orc.conv2d_nhwc(x, w, b, stride=s, padding=p)
    if relu:
        ref = orc.relu(ref)
    del x
    for mode, y in outs.items():
        assert y.shape == (BATCH, oh, oh, cout)
        for i0 in range(0, BATCH, 16):  # in image blocks, to bound the float64 temporaries
            check_bf16(y[i0:i0 + 16], ref[i0:i0 + 16], f"{name} {mode}: images {i0}..{i0 + 15}")
