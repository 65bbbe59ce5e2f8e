"""Fusion of operator chains onto the fused entry points.

A graph here is a list of nodes in topological order, each with an op name,
the indices of its input nodes, attributes and a dtype: the shape of the
reference's teeny_core Graph (GraphNode { op, inputs, dtype }).  Two
rewrites, each to a fixed point:

1. Pointwise chains, the Anduin pass (kernels/teeny-kernels/src/graph/
   optimizer/anduin.rs:27-60, fuse_pointwise_chain_pass): a unary pointwise
   node (or chain) whose single input is another unary pointwise node (or
   chain) that nothing else consumes, of the same dtype, absorbs it into one
   PointwiseFuse node whose members run in order (graph/optimizer/ops/
   pointwise_fuse.rs:73-120).  Members are the activations with a fused
   kernel: relu, gelu, silu, sigmoid, tanh.
2. Epilogues: an activation (or the first member of a chain) whose producer
   is consumed by nothing else moves into that producer's epilogue, and a
   BatchNorm after a conv becomes the conv's per-channel affine:
     conv2d -> batchnorm [-> act]        conv2d_bn_act (nn/fused/conv2d_bn_silu.rs)
     conv2d -> act                       conv2d with its epilogue activation
     layer_norm | rms_norm -> act        norm_act
     w8a16_linear -> act                 w8a16_linear with ACT
   where act is relu, gelu or silu (the activations the epilogues apply).

`run(graph, feeds)` executes a graph through the library's entry points, so
a fused graph can be checked against the graph it came from.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import kernels as K
from .runtime import Buffer, Stream

UNARY = ("relu", "gelu", "silu", "sigmoid", "tanh")
EPILOGUE_ACTS = ("relu", "gelu", "silu")
PRODUCERS = ("conv2d", "conv2d_bn_act", "layer_norm", "rms_norm", "w8a16_linear")


@dataclass
class Node:
    op: str
    inputs: List[int] = field(default_factory=list)
    attrs: Dict = field(default_factory=dict)
    dtype: str = "bf16"


def consumers(graph: Sequence[Node]) -> List[int]:
    n = [0] * len(graph)
    for node in graph:
        for i in node.inputs:
            n[i] += 1
    return n


def _members(node: Node) -> Optional[List[str]]:
    """A node's pointwise members, or None if it is not pointwise-fusable."""
    if node.op in UNARY:
        return [node.op]
    if node.op == "pointwise_fuse":
        return list(node.attrs["members"])
    return None


def _rebuild(graph: Sequence[Node], dead: Sequence[bool], override: Dict[int, Node]) -> List[Node]:
    """Drops dead nodes, applies overrides and renumbers the inputs."""
    new_index, out = {}, []
    for i, node in enumerate(graph):
        if dead[i]:
            continue
        new_index[i] = len(out)
        out.append(copy.copy(override.get(i, node)))
    for node in out:
        node.inputs = [new_index[i] for i in node.inputs]
    return out


def fuse_pointwise_chains(graph: Sequence[Node]) -> List[Node]:
    """The Anduin pass: one merge per sweep (the reference's loop), repeated
    until nothing changes."""
    graph = list(graph)
    while True:
        n_cons = consumers(graph)
        changed = False
        for child, node in enumerate(graph):
            child_members = _members(node)
            if child_members is None or len(node.inputs) != 1:
                continue
            parent = node.inputs[0]
            if n_cons[parent] != 1 or graph[parent].dtype != node.dtype:
                continue
            parent_members = _members(graph[parent])
            if parent_members is None:
                continue
            members = parent_members + child_members
            if len(members) > 8:
                continue
            fused = Node("pointwise_fuse", list(graph[parent].inputs), {"members": members}, node.dtype)
            dead = [False] * len(graph)
            dead[parent] = True
            graph = _rebuild(graph, dead, {child: fused})
            changed = True
            break
        if not changed:
            return graph


def fuse_epilogues(graph: Sequence[Node]) -> List[Node]:
    """Moves BatchNorm and activations into their producers' epilogues."""
    graph = list(graph)
    while True:
        n_cons = consumers(graph)
        changed = False
        for child, node in enumerate(graph):
            if len(node.inputs) != 1:
                continue
            parent = node.inputs[0]
            pnode = graph[parent]
            if n_cons[parent] != 1 or pnode.dtype != node.dtype:
                continue
            fused, rest = None, None
            if node.op == "batchnorm" and pnode.op == "conv2d" and pnode.attrs.get("act") is None \
                    and pnode.attrs.get("bias") is None:
                scale, shift = K.fold_batchnorm(node.attrs["gamma"], node.attrs["beta"], node.attrs["mean"],
                                                node.attrs["var"], node.attrs.get("eps", 1e-5))
                attrs = dict(pnode.attrs)
                attrs.update(bn_scale=scale, bn_shift=shift, act=None)
                fused = Node("conv2d_bn_act", list(pnode.inputs), attrs, node.dtype)
            else:
                members = _members(node)
                if members is None or members[0] not in EPILOGUE_ACTS or pnode.op not in PRODUCERS \
                        or pnode.attrs.get("act") is not None:
                    continue
                attrs = dict(pnode.attrs)
                attrs["act"] = members[0]
                fused = Node(pnode.op, list(pnode.inputs), attrs, node.dtype)
                tail = members[1:]
                if len(tail) == 1:
                    rest = Node(tail[0], [], {}, node.dtype)
                elif tail:
                    rest = Node("pointwise_fuse", [], {"members": tail}, node.dtype)
            if rest is None:
                dead = [False] * len(graph)
                dead[parent] = True
                graph = _rebuild(graph, dead, {child: fused})
            else:
                # the producer absorbs the first member; the child keeps the rest
                rest.inputs = [parent]
                graph = _rebuild(graph, [False] * len(graph), {parent: fused, child: rest})
            changed = True
            break
        if not changed:
            return graph


def optimize(graph: Sequence[Node]) -> List[Node]:
    """Pointwise chains first (Anduin), then epilogues."""
    return fuse_epilogues(fuse_pointwise_chains(graph))


# ── execution ────────────────────────────────────────────────────────────────


def _dev_f32(dev, a):
    return a if isinstance(a, Buffer) else dev.upload(np.ascontiguousarray(a, np.float32))


def run(graph: Sequence[Node], feeds: Dict[int, Buffer], dev, stream: Optional[Stream] = None,
        keep_scratch: bool = False) -> List[Optional[Buffer]]:
    """Runs every node on the device; returns each node's output buffer.
    `feeds` maps "input" node indices to buffers.  Chains keep their member
    outputs (the backward's scratch) when keep_scratch is set."""
    out: List[Optional[Buffer]] = [None] * len(graph)
    for i, node in enumerate(graph):
        a = node.attrs
        xs = [out[j] for j in node.inputs]
        if node.op == "input":
            out[i] = feeds[i]
        elif node.op in UNARY:
            y = K.pointwise_chain(xs[0], [node.op], stream=stream) if node.op in ("sigmoid", "tanh") else \
                getattr(K, node.op)(xs[0], stream=stream)
            out[i] = y
        elif node.op == "pointwise_fuse":
            scratch = [Buffer(xs[0].dtype, xs[0].shape) for _ in a["members"][:-1]] if keep_scratch else None
            out[i] = K.pointwise_chain(xs[0], a["members"], scratch=scratch, stream=stream)
            if keep_scratch:
                a["scratch_buffers"] = scratch
        elif node.op == "conv2d":
            out[i] = K.conv2d(xs[0], a["weight"], a.get("bias"), a.get("stride", 1), a.get("padding", 0),
                              a.get("groups", 1), a.get("act"), a.get("layout", "nchw"), stream=stream)
        elif node.op == "conv2d_bn_act":
            out[i] = K.conv2d_bn_act(xs[0], a["weight"], _dev_f32(dev, a["bn_scale"]), _dev_f32(dev, a["bn_shift"]),
                                     a.get("stride", 1), a.get("padding", 0), a.get("groups", 1), a.get("act"),
                                     a.get("layout", "nchw"), stream=stream)
        elif node.op == "batchnorm":
            # unfused: the affine as a conv-free per-channel op is not a kernel of
            # this library; a graph keeps BatchNorm only behind a conv, where the
            # epilogue pass folds it
            raise ValueError("batchnorm must follow a conv2d (run optimize() first)")
        elif node.op in ("layer_norm", "rms_norm"):
            rms = node.op == "rms_norm"
            act = a.get("act")
            if act is None:
                out[i] = (K.rms_norm(xs[0], a["weight"], a.get("eps", 1e-8), stream=stream) if rms else
                          K.layer_norm(xs[0], a["weight"], a["bias"], a.get("eps", 1e-5), stream=stream))
            else:
                out[i] = K.norm_act(xs[0], a["weight"], None if rms else a["bias"], a.get("eps", 1e-8 if rms else 1e-5),
                                    rms, act, stream=stream)
        elif node.op == "w8a16_linear":
            out[i] = K.w8a16_linear(xs[0], a["qweight"], a["scale"], a.get("bias"), act=a.get("act"), stream=stream)
        else:
            raise ValueError(f"fusion.run: no lowering for op {node.op!r}")
    return out
