"""Host-side contract: RuntimeOp packing/grids against the reference impls,
bf16 conversion, and the synthetic input generator."""
import math

import numpy as np
import pytest

from teenygrad_amd import dtypes, kernels, synthetic
from teenygrad_amd import kernels as K
from teenygrad_amd.kernels import RecordingVisitor


def pack(op, inputs, params, output, output_shape):
    v = RecordingVisitor()
    op.pack_args(inputs, params, output, output_shape, op.forward_output_row_stride(output_shape), v)
    return v.args


def test_conv2d_bias_runtime_op_matches_reference():
    # conv2d.rs:766-820: params [[Cout, Cin/G, KH, KW], [Cout]], args
    # (x, w, bias, y, B, C_IN, C_OUT, H, W, OH, OW), grid B*Cout*OH*ceil(OW/BLOCK_OW)
    op = kernels.Conv2dBiasForward(3, 3, 1, 1, 1, 1, 2, 16)
    ish, osh = [2, 4, 9, 9], [2, 6, 9, 9]
    assert op.param_shapes([ish], osh) == [[6, 2, 3, 3], [6]]
    assert op.param_names() == ("weight", "bias")
    assert op.entry_point_name() == "conv2d_bias_forward_entry_point"
    args = pack(op, [(1, ish)], [2, 3], 4, osh)
    assert args == [("ptr", 1), ("ptr", 2), ("ptr", 3), ("ptr", 4), ("i32", 2), ("i32", 4),
                    ("i32", 6), ("i32", 9), ("i32", 9), ("i32", 9), ("i32", 9)]
    assert op.grid(osh) == (2 * 6 * 9 * 1, 1, 1)
    assert op.const_generics() == (3, 3, 1, 1, 1, 1, 2, 16)


def test_conv2d_runtime_op_matches_reference():
    # conv2d.rs:523-618
    op = kernels.Conv2dForward(3, 3, block_ow=8)
    args = pack(op, [(10, [1, 2, 8, 8])], [11], 12, [1, 4, 6, 6])
    assert [a[0] for a in args] == ["ptr"] * 3 + ["i32"] * 7
    assert args[3:] == [("i32", 1), ("i32", 2), ("i32", 4), ("i32", 8), ("i32", 8), ("i32", 6), ("i32", 6)]
    assert op.grid([1, 4, 6, 6]) == (1 * 4 * 6 * 1, 1, 1)


def test_layernorm_runtime_op_matches_reference():
    # layernorm.rs:486-561: (x, y, weight, bias, M, N, eps), grid [M]
    op = kernels.LayerNormForwardInferenceRuntimeOp(1024, 1e-5)
    shape = [4, 16, 128]
    assert op.param_shapes([shape], shape) == [[128], [128]]
    args = pack(op, [(1, shape)], [2, 3], 4, shape)
    assert args[:4] == [("ptr", 1), ("ptr", 4), ("ptr", 2), ("ptr", 3)]
    assert args[4:6] == [("i32", 64), ("i32", 128)]
    assert args[6][0] == "f32" and math.isclose(args[6][1], 1e-5, rel_tol=1e-6)
    assert op.grid(shape) == (64, 1, 1)


def test_rmsnorm_runtime_op():
    # rmsnorm.rs:39-47 argument order (x, y, weight, rrms, M, N, eps)
    op = kernels.RmsNormForwardRuntimeOp()
    assert op.param_shapes([[16, 128]], [16, 128]) == [[128], [16]]
    args = pack(op, [(1, [16, 128])], [2, 3], 4, [16, 128])
    assert args[:4] == [("ptr", 1), ("ptr", 4), ("ptr", 2), ("ptr", 3)]
    assert op.grid([16, 128]) == (16, 1, 1)


@pytest.mark.parametrize("cls,name", [(kernels.ReluForward, "relu_forward"),
                                      (kernels.GeluForward, "gelu_forward"),
                                      (kernels.SiluForward, "silu_forward")])
def test_elementwise_runtime_ops(cls, name):
    # relu.rs:119-180 etc: (x, y, n), grid ceil(n / BLOCK_SIZE)
    op = cls(1024)
    assert op.name == name and op.param_shapes([[3, 1000]], [3, 1000]) == []
    assert pack(op, [(5, [3, 1000])], [], 6, [3, 1000]) == [("ptr", 5), ("ptr", 6), ("i32", 3000)]
    assert op.grid([3, 1000]) == (3, 1, 1)


@pytest.mark.parametrize("cls,bname,saved", [(kernels.ReluForward, "relu_backward", "output"),
                                              (kernels.GeluForward, "gelu_backward", "input"),
                                              (kernels.SiluForward, "silu_backward", "input")])
def test_elementwise_backward_hooks(cls, bname, saved):
    # relu.rs:148-180, gelu.rs:287-317, sigmoid.rs:418-448: (dy, y | x, dx, n)
    op = cls(1024)
    assert op.has_backward() and op.backward_entry_point_name() == f"{bname}_entry_point"
    v = RecordingVisitor()
    op.pack_backward_args([(5, [3, 1000])], [], 6, [3, 1000], 7, 1000, [8], [], v)
    want_saved = 6 if saved == "output" else 5
    assert v.args == [("ptr", 7), ("ptr", want_saved), ("ptr", 8), ("i32", 3000)]
    assert op.backward_grid([[3, 1000]], [3, 1000]) == (3, 1, 1)


def test_flash_attention_launch_contract():
    # tests/test_flash_attn2.rs:135-162: grid (N_CTX, BH, 1), args (q,k,v,o,l,nq,nk,scale,-inf)
    op = kernels.FlashAttention2Forward(64, 0.125)
    args = pack(op, [(1, [4, 8, 64]), (2, [4, 8, 64]), (3, [4, 8, 64])], [5], 4, [4, 8, 64])
    assert args[:5] == [("ptr", i) for i in (1, 2, 3, 4, 5)]
    assert args[5:7] == [("i32", 8), ("i32", 8)]
    assert args[7] == ("f32", 0.125) and args[8] == ("f32", float("-inf"))
    assert op.grid([4, 8, 64]) == (8, 4, 1)


def test_linear_runtime_op_matches_reference():
    # linear.rs:250-320
    op = kernels.LinearForward(use_bias=False)
    assert op.param_shapes([[64, 32]], [64, 48]) == [[48, 32]]
    args = pack(op, [(1, [64, 32])], [2], 3, [64, 48])
    assert args[2] == ("ptr", None)
    assert [a[1] for a in args[4:]] == [64, 48, 32, 32, 1, 32, 1, 48, 1]
    assert op.grid([64, 48]) == (1, 1, 1)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 10000) * 10.0 ** rng.integers(-30, 30, 10000),
                        [0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(dtypes.to_bf16(x), want)
    np.testing.assert_array_equal(dtypes.from_bf16(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())
    assert np.isnan(dtypes.from_bf16(dtypes.to_bf16(np.array([np.nan], np.float32))))[0]


def test_synthetic_is_seeded():
    a = synthetic.normal(123, (1000,))
    np.testing.assert_array_equal(a, synthetic.normal(123, (1000,)))
    assert not np.array_equal(a, synthetic.normal(124, (1000,)))
    big = synthetic.normal(5, (1 << 23) + 17, mean=1.0, std=0.02)
    assert big.dtype == np.float32
    assert abs(float(big.mean()) - 1.0) < 1e-4 and abs(float(big.std()) - 0.02) < 1e-4
    u = synthetic.uniform(9, (100000,), -1, 1)
    assert u.min() >= -1 and u.max() <= 1 and abs(float(u.mean())) < 1e-2
    assert synthetic.workload_seed(1, 0) != synthetic.workload_seed(1, 1) != synthetic.workload_seed(2, 0)


# ── host-side shape rules of the Buffer wrappers (no device needed) ─────────


def test_w8a16_rejects_flat_weight():
    # a flattened [N*K] int8 weight must not be read as N*K output channels
    with pytest.raises(ValueError):
        kernels.w8a16_dims((64, 512), (256 * 512,), (256,))
    with pytest.raises(ValueError):
        kernels.w8a16_dims((64, 512), (256, 512), (255,))
    assert kernels.w8a16_dims((64, 512), (256, 512), (256,), (256,)) == (64, 256, 512)


def test_linear_and_conv_shape_rules():
    with pytest.raises(ValueError):
        kernels.linear_dims((4, 8), (3, 7))
    assert kernels.linear_dims((4, 8), (3, 8), (3,)) == (4, 3, 8)
    d = kernels.conv2d_dims((2, 4, 9, 9), (6, 2, 3, 3), 1, 1, 2, "nchw", (6,))
    assert d[:7] == (2, 4, 6, 9, 9, 9, 9)
    d = kernels.conv2d_dims((2, 9, 9, 4), (6, 3, 3, 4), (2, 2), (1, 1), 1, "nhwc")
    assert d[:7] == (2, 4, 6, 9, 9, 5, 5)
    for bad in [((2, 4, 9, 9), (6, 4, 3, 3), 1, 1, 2, "nchw"),   # weight Cin/G mismatch
                ((2, 4, 9, 9), (5, 2, 3, 3), 1, 1, 2, "nchw"),   # groups do not divide Cout
                ((1, 4, 2, 2), (4, 4, 5, 5), 1, 0, 1, "nchw")]:  # kernel larger than input
        with pytest.raises(ValueError):
            kernels.conv2d_dims(*bad)


def test_attention_and_norm_shape_rules():
    assert kernels.attention_dims((4, 8, 64), (4, 16, 64), (4, 16, 64), (4, 8)) == (4, 8, 16, 64)
    with pytest.raises(ValueError):
        kernels.attention_dims((4, 8, 64), (4, 16, 64), (4, 15, 64))
    with pytest.raises(ValueError):
        kernels.attention_dims((4, 8, 64), (2, 16, 64), (2, 16, 64))
    assert kernels.norm_dims((16, 4, 128), (128,), (128,), (64,)) == (64, 128)
    with pytest.raises(ValueError):
        kernels.norm_dims((16, 128), (127,))


def test_runtime_op_buffer_check_uses_param_shapes():
    class FakeBuf(kernels.Buffer):
        def __init__(self, n):  # no device allocation
            self.numel, self.ptr, self.shape = n, 0x1000, (n,)

        def __del__(self):
            pass

    op = kernels.Conv2dBiasForward(3, 3, 1, 1, 1, 1, 1, 16)
    ok = dict(inputs=[(FakeBuf(2 * 4 * 81), [2, 4, 9, 9])], output=FakeBuf(2 * 6 * 81),
              output_shape=[2, 6, 9, 9])
    op.check_buffers(params=[FakeBuf(6 * 4 * 9), FakeBuf(6)], **ok)
    with pytest.raises(ValueError):
        op.check_buffers(params=[FakeBuf(6 * 4 * 9), FakeBuf(5)], **ok)
    with pytest.raises(ValueError):
        op.check_buffers(inputs=[(FakeBuf(10), [2, 4, 9, 9])], params=[FakeBuf(216), FakeBuf(6)],
                         output=ok["output"], output_shape=ok["output_shape"])


def test_lowering_runtime_ops_for_reference_todo_arms():
    # argument lists the new dispatch names read (dispatch.cpp), packed by the mirrors
    rv = K.RecordingVisitor()
    mha = K.MultiHeadAttentionRuntimeOp(8, 2, 128, causal=True)
    mha.pack_args([(1, [16, 64, 128]), (2, [4, 64, 128]), (3, [4, 64, 128])], [4], 5, [16, 64, 128], 128, rv)
    assert [k for k, _ in rv.args] == ["ptr"] * 5 + ["i32", "i32", "f32", "f32"]
    assert mha.const_generics() == (128, 1, 8, 2) and mha.grid([16, 64, 128]) == (64, 16, 1)
    assert mha.entry_point_name() == "multi_head_attention_forward_entry_point"
    with pytest.raises(ValueError):
        K.MultiHeadAttentionRuntimeOp(6, 4, 64)
    rv = K.RecordingVisitor()
    lin = K.W8A16LinearRuntimeOp(False, "gelu")
    lin.pack_args([(1, [10, 32])], [2, 3], 4, [10, 48], 48, rv)
    assert rv.args == [("ptr", 1), ("ptr", 2), ("ptr", 3), ("ptr", None), ("ptr", 4), ("i32", 10), ("i32", 48),
                       ("i32", 32)]
    assert lin.param_shapes([[10, 32]], [10, 48]) == [[48, 32], [48]]
    rv = K.RecordingVisitor()
    cv = K.W8A16Conv2dRuntimeOp(3, 3, 1, 1, 1, 1, 1, 16, True, "relu")
    cv.pack_args([(1, [2, 8, 9, 16])], [2, 3, 5], 4, [2, 8, 9, 24], 24, rv)
    assert [v for _, v in rv.args] == [1, 2, 3, 5, 4, 2, 16, 24, 8, 9, 8, 9]
    assert cv.const_generics() == (3, 3, 1, 1, 1, 1, 1, 16, 1, 1)
    assert cv.param_shapes([[2, 8, 9, 16]], [2, 8, 9, 24]) == [[24, 3, 3, 16], [24], [24]]
    rv = K.RecordingVisitor()
    qop = K.QuantizeAffineRuntimeOp("group", 1, 8, False, 4)
    qop.pack_args([(1, [3, 16])], [2, 3], 4, [3, 16], 16, rv)
    assert rv.args == [("ptr", 1), ("ptr", 4), ("ptr", 2), ("ptr", 3), ("ptr", None), ("i32", 2), ("i64", 3),
                       ("i64", 16)]
    assert qop.const_generics() == (2, 1, 8, 0, 4)
    rv = K.RecordingVisitor()
    K.DequantizeAffineRuntimeOp("channel", 0).pack_args([(1, [5, 7])], [2, 3], 4, [5, 7], 7, rv)
    assert [k for k, _ in rv.args] == ["ptr"] * 4 + ["i32", "i64", "i64"]
