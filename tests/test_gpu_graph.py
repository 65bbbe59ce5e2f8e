"""GPU: operators captured into a HIP graph (teeny_hip_stream_begin_capture /
end_capture / graph_launch) replay to exactly the eager results.

The reference executor captures a whole model into one CUDA graph
(LoadedModel::capture_graph, drivers/teeny-cuda/src/model/mod.rs:1245-1640).
Here a sequence covering every kernel family — LayerNorm -> GELU, a split-K
conv using the stream workspace, a space-to-depth stem conv, a W8A16 GEMM
(int8 weights converted in registers), causal attention — is captured once and
replayed several times.  Before every replay the outputs are overwritten
(eagerly, outside the graph), other eager work runs on the same stream, and
the stream is synchronized; after it, every output must equal the eager
result bit for bit."""
import numpy as np
import pytest

import teenygrad_amd as tg
from gpu_util import check_bf16
from teenygrad_amd import kernels as K
from teenygrad_amd._lib import check, lib
from teenygrad_amd.dtypes import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def up(dev, a):
    return dev.upload(to_bf16(a), tg.bf16)


def test_graph_replays_equal_eager(dev, orc):
    rng = np.random.default_rng(99)
    stream = tg.Stream.create()
    # LayerNorm -> GELU, bf16 [512, 4096]
    x = from_bf16(to_bf16(rng.standard_normal((512, 4096), dtype=np.float32)))
    g = np.ones(4096, np.float32)
    b = np.zeros(4096, np.float32)
    xb, gb, bb = up(dev, x), up(dev, g), up(dev, b)
    ln, ge = tg.Buffer(tg.bf16, x.shape), tg.Buffer(tg.bf16, x.shape)
    # split-K 3x3 conv (512 -> 512 at 7x7) and the 3-channel stride-2 stem
    cx = up(dev, rng.random((8, 7, 7, 512), dtype=np.float32))
    cw = up(dev, rng.standard_normal((512, 3, 3, 512), dtype=np.float32) * np.float32(0.02))
    cb = up(dev, rng.normal(0, 0.01, 512).astype(np.float32))
    cy = tg.Buffer(tg.bf16, (8, 7, 7, 512))
    sx = up(dev, rng.random((4, 64, 64, 3), dtype=np.float32))
    sw = up(dev, rng.standard_normal((64, 7, 7, 3), dtype=np.float32) * np.float32(0.1))
    sb = up(dev, rng.normal(0, 0.01, 64).astype(np.float32))
    sy = tg.Buffer(tg.bf16, (4, 32, 32, 64))
    # W8A16 GEMM at M = 4096 (the 256 x 256 LDS-DMA kernel) and a
    # decode-sized one (split-K partials in the workspace)
    wf = rng.normal(0, 0.02, (1024, 1024)).astype(np.float32)
    q, s, _, _ = K.quantize_affine(dev.upload(wf), [1024, 1024], "channel", 0)
    lx = up(dev, rng.standard_normal((4096, 1024), dtype=np.float32))
    ly = tg.Buffer(tg.bf16, (4096, 1024))
    dx_ = up(dev, rng.standard_normal((16, 1024), dtype=np.float32))
    dy_ = tg.Buffer(tg.bf16, (16, 1024))
    # causal attention
    qa, ka, va = (up(dev, rng.standard_normal((4, 300, 128), dtype=np.float32)) for _ in range(3))
    oa = tg.Buffer(tg.bf16, (4, 300, 128))
    need = max(K.conv2d_workspace_size((8, 7, 7, 512), (512, 3, 3, 512), 1, 1, 1, tg.bf16),
               K.conv2d_workspace_size((4, 64, 64, 3), (64, 7, 7, 3), 2, 3, 1, tg.bf16),
               K.linear_workspace_size(4096, 1024, 1024, tg.i8), K.linear_workspace_size(16, 1024, 1024, tg.i8))
    ws = dev.buffer(tg.i8, (need,))
    stream.set_workspace(ws)
    outs = [ln, ge, cy, sy, ly, dy_, oa]

    def sequence():
        K.layer_norm(xb, gb, bb, 1e-5, y=ln, stream=stream)
        K.gelu(ln, y=ge, stream=stream)
        K.conv2d(cx, cw, cb, 1, 1, 1, "relu", "nhwc", y=cy, stream=stream)
        K.conv2d(sx, sw, sb, 2, 3, 1, "relu", "nhwc", y=sy, stream=stream)
        K.w8a16_linear(lx, q, s, act="silu", y=ly, stream=stream)
        K.w8a16_linear(dx_, q, s, y=dy_, stream=stream)
        K.flash_attention(qa, ka, va, None, True, o=oa, stream=stream)

    sequence()
    stream.synchronize()
    eager = [o.to_host() for o in outs]
    # the eager results are right (spot checks against the oracle)
    check_bf16(ln.to_host()[:8], orc.layer_norm(x[:8], g, b, 1e-5), "layernorm")
    stream.begin_capture()
    sequence()
    graph = stream.end_capture()
    junk = tg.Buffer(tg.bf16, x.shape)
    for replay in range(4):
        print(f"[graph] replay {replay}", flush=True)
        for o in outs:  # overwrite the outputs, outside the graph
            check(lib.teeny_hip_memset(o.ptr, 0x7F, o.nbytes, stream.handle))
        K.silu(xb, y=junk, stream=stream)  # eager work between replays
        stream.synchronize()
        graph.launch(stream)
        stream.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            np.testing.assert_array_equal(o.to_host(), e, err_msg=f"replay {replay}, output {i}")
    graph.destroy()
    stream.set_workspace(None)
    stream.destroy()
