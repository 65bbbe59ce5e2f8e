"""The fusion passes without a GPU: Anduin's pointwise-chain rule
(kernels/teeny-kernels/src/graph/optimizer/anduin.rs:27-60) and the epilogue
mapping, on small graphs; the PointwiseFuse RuntimeOp's argument lists
(graph/optimizer/ops/pointwise_fuse.rs:155-268)."""
import numpy as np

from teenygrad_amd import _lib
from teenygrad_amd import kernels as K
from teenygrad_amd.fusion import Node, consumers, fuse_epilogues, fuse_pointwise_chains, optimize


def ops(graph):
    return [(n.op, n.inputs, n.attrs.get("members"), n.attrs.get("act")) for n in graph]


def test_chain_collapses_to_one_node():
    g = [Node("input"), Node("relu", [0]), Node("sigmoid", [1]), Node("tanh", [2])]
    out = fuse_pointwise_chains(g)
    assert ops(out) == [("input", [], None, None), ("pointwise_fuse", [0], ["relu", "sigmoid", "tanh"], None)]


def test_shared_parent_blocks_fusion():
    # relu feeds two nodes: it must stay materialized (anduin.rs: n_consumers[parent] == 1)
    g = [Node("input"), Node("relu", [0]), Node("sigmoid", [1]), Node("tanh", [1])]
    assert ops(fuse_pointwise_chains(g)) == ops(g)


def test_dtype_boundary_blocks_fusion():
    g = [Node("input", dtype="f32"), Node("relu", [0], dtype="f32"), Node("sigmoid", [1], dtype="bf16")]
    assert ops(fuse_pointwise_chains(g)) == ops(g)


def test_non_pointwise_breaks_chains():
    g = [Node("input"), Node("relu", [0]), Node("sigmoid", [1]), Node("layer_norm", [2]), Node("tanh", [3]),
         Node("silu", [4])]
    out = fuse_pointwise_chains(g)
    assert [n.op for n in out] == ["input", "pointwise_fuse", "layer_norm", "pointwise_fuse"]
    assert out[1].attrs["members"] == ["relu", "sigmoid"] and out[3].attrs["members"] == ["tanh", "silu"]
    assert out[3].inputs == [2]


def test_conv_bn_act_epilogue():
    gamma, beta, mean, var = np.ones(4), np.zeros(4), np.zeros(4), np.ones(4)
    g = [Node("input"), Node("conv2d", [0], {"weight": None}), Node("batchnorm", [1], {
        "gamma": gamma, "beta": beta, "mean": mean, "var": var}), Node("silu", [2])]
    out = optimize(g)
    assert [(n.op, n.attrs.get("act")) for n in out] == [("input", None), ("conv2d_bn_act", "silu")]
    assert out[1].inputs == [0]
    np.testing.assert_allclose(out[1].attrs["bn_scale"], 1 / np.sqrt(1 + 1e-5), rtol=1e-6)


def test_norm_absorbs_first_chain_member():
    # layer_norm -> gelu -> sigmoid: Anduin makes [gelu, sigmoid]; the norm takes gelu
    g = [Node("input"), Node("layer_norm", [0], {"weight": None, "bias": None}), Node("gelu", [1]),
         Node("sigmoid", [2])]
    out = optimize(g)
    assert ops(out) == [("input", [], None, None), ("layer_norm", [0], None, "gelu"), ("sigmoid", [1], None, None)]
    # three members: the rest stays a chain
    g.append(Node("tanh", [3]))
    out = optimize(g)
    assert ops(out)[-1] == ("pointwise_fuse", [1], ["sigmoid", "tanh"], None)


def test_epilogue_needs_single_consumer_and_supported_act():
    g = [Node("input"), Node("conv2d", [0], {"weight": None}), Node("relu", [1]), Node("relu", [1])]
    assert ops(fuse_epilogues(g)) == ops(g)
    g = [Node("input"), Node("conv2d", [0], {"weight": None}), Node("sigmoid", [1])]
    assert ops(fuse_epilogues(g)) == ops(g)  # no epilogue applies sigmoid
    g = [Node("input"), Node("conv2d", [0], {"weight": None, "act": "relu"}), Node("relu", [1])]
    assert ops(fuse_epilogues(g)) == ops(g)  # the epilogue slot is taken


def test_consumer_counts():
    g = [Node("input"), Node("relu", [0]), Node("tanh", [0]), Node("silu", [1])]
    assert consumers(g) == [2, 1, 0, 0]


def test_pointwise_fuse_runtime_op_args():
    op = K.PointwiseFuse(["relu", "sigmoid", "tanh"])
    assert op.entry_point_name() == "pointwise_fuse_relu_sigmoid_tanh_entry_point"
    assert op.backward_entry_point_name() == "pointwise_fuse_relu_sigmoid_tanh_backward_entry_point"
    assert op.param_shapes([[4, 6]], [4, 6]) == [[24], [24]]
    assert op.has_backward() and not K.PointwiseFuse(["gelu", "relu"]).has_backward()
    p = K.DispatchPacker()
    op.pack_args([(0x1000, [4, 6])], [0x2000, 0x3000], 0x4000, [4, 6], 6, p)
    assert [a.kind for a in p.args] == [_lib.ARG_PTR] * 4 + [_lib.ARG_I32]
    assert [a.v.ptr for a in p.args[:4]] == [0x1000, 0x4000, 0x2000, 0x3000]
    assert p.args[-1].v.i32 == 24
    q = K.DispatchPacker()
    op.pack_backward_args([(0x1000, [4, 6])], [0x2000, 0x3000], 0x4000, [4, 6], 0x5000, 6, [0x6000], [], q)
    assert [a.v.ptr for a in q.args[:5]] == [0x5000, 0x4000, 0x6000, 0x2000, 0x3000]
    assert op.grid([4, 6]) == (1, 1, 1)


def test_conv_bn_silu_runtime_ops():
    op = K.Conv2dBnSiluForward(3, 3, 1, 1, 1, 1)
    assert op.param_shapes([[2, 8, 10, 10]], [2, 16, 10, 10]) == [[16, 8, 3, 3], [16], [16]]
    gemm = K.Conv2dBnSiluGemmForward(32, 32, 32, 8)
    assert gemm.forward_output_row_stride([2, 16, 7, 7]) == 64
    assert gemm.grid([2, 16, 7, 7]) == (2 * 2 * 1, 1, 1)
    tiled = K.Conv2dBnSiluTiledForward(3, 3, 1, 1, 1, 1, 16, 16)
    assert tiled.forward_output_row_stride([1, 8, 40, 40]) == 48
    assert tiled.grid([1, 8, 40, 40]) == (40 * 1 * 3, 1, 1)
