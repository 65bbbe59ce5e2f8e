"""Host-side mirror of teeny-kernels' operator contract, dispatching to HIP.

Two layers:

* ``RuntimeOp`` subclasses reproduce the reference's per-kernel RuntimeOp
  impls — ``param_shapes``, ``param_names``, ``pack_args`` (argument kinds and
  order exactly as the reference visits them), ``grid`` and the
  ``"{name}_entry_point"`` symbol — and ``launch`` hands the packed list to
  ``teeny_dispatch`` in place of cuLaunchKernel.  Reference:
  core/teeny-core/src/model/mod.rs:78-331 (RuntimeOp),
  core/teeny-core/src/device/program.rs:22-46 (ArgVisitor), the impls cited
  on each class, and the executor loop that calls them,
  drivers/teeny-cuda/src/model/mod.rs:524-700.

* Functions (``relu``, ``layer_norm``, ``conv2d``, ``flash_attention`` ...)
  call the typed entry points of include/teeny_hip.h directly on
  ``Buffer`` objects, with this library's extensions (bf16, NHWC, causal,
  fused activations, W8A16).
"""
from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import _lib
from ._lib import check, lib
from .dtypes import DType, bf16, f32, from_any, i8
from .runtime import Buffer, Stream, _h

# ── ArgVisitor (core/teeny-core/src/device/program.rs:22-46) ────────────────


class ArgVisitor:
    def visit_ptr(self, ptr): raise NotImplementedError
    def visit_bool(self, v: bool): raise NotImplementedError
    def visit_i32(self, v: int): raise NotImplementedError
    def visit_i64(self, v: int): raise NotImplementedError
    def visit_u32(self, v: int): raise NotImplementedError
    def visit_f32(self, v: float): raise NotImplementedError
    def visit_f64(self, v: float): raise NotImplementedError


def _addr(p) -> Optional[int]:
    if p is None:
        return None
    if isinstance(p, Buffer):
        return p.ptr
    return int(p)


class RecordingVisitor(ArgVisitor):
    """Records (kind, value) pairs; used to compare packing with the reference."""

    def __init__(self):
        self.args: List[Tuple[str, object]] = []

    def visit_ptr(self, ptr): self.args.append(("ptr", _addr(ptr)))
    def visit_bool(self, v): self.args.append(("bool", bool(v)))
    def visit_i32(self, v): self.args.append(("i32", int(v)))
    def visit_i64(self, v): self.args.append(("i64", int(v)))
    def visit_u32(self, v): self.args.append(("u32", int(v)))
    def visit_f32(self, v): self.args.append(("f32", float(v)))
    def visit_f64(self, v): self.args.append(("f64", float(v)))


class DispatchPacker(ArgVisitor):
    """Builds the teeny_arg array that teeny_dispatch consumes."""

    def __init__(self):
        self.args: List[_lib.TeenyArg] = []

    def _push(self, kind, field, value):
        a = _lib.TeenyArg()
        a.kind = kind
        setattr(a.v, field, value)
        self.args.append(a)

    def visit_ptr(self, ptr): self._push(_lib.ARG_PTR, "ptr", _addr(ptr))
    def visit_bool(self, v): self._push(_lib.ARG_BOOL, "b", int(bool(v)))
    def visit_i32(self, v): self._push(_lib.ARG_I32, "i32", int(v))
    def visit_i64(self, v): self._push(_lib.ARG_I64, "i64", int(v))
    def visit_u32(self, v): self._push(_lib.ARG_U32, "u32", int(v))
    def visit_f32(self, v): self._push(_lib.ARG_F32, "f32", float(v))
    def visit_f64(self, v): self._push(_lib.ARG_F64, "f64", float(v))

    def array(self):
        arr = (_lib.TeenyArg * max(1, len(self.args)))(*self.args)
        return arr, len(self.args)


# ── RuntimeOp (core/teeny-core/src/model/mod.rs:78-331) ─────────────────────


def _prod(s: Sequence[int]) -> int:
    return int(np.prod(s)) if len(s) else 1


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


class RuntimeOp:
    name: str = ""

    def const_generics(self) -> Tuple[int, ...]:
        return ()

    def entry_point_name(self) -> str:  # Kernel::entry_point_name, program.rs:212-216
        return f"{self.name}_entry_point"

    def n_activation_inputs(self) -> int:
        return 1

    def param_shapes(self, input_shapes, output_shape) -> List[List[int]]:
        return []

    def param_names(self) -> Tuple[str, ...]:
        return ()

    def forward_output_row_elems(self, output_shape) -> int:
        return int(output_shape[-1]) if len(output_shape) else 1

    def forward_output_row_stride(self, output_shape) -> int:
        return self.forward_output_row_elems(output_shape)

    def compute_concrete_output_shape(self, input_shapes, resolved):
        return list(resolved)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        raise NotImplementedError

    def grid(self, output_shape) -> Tuple[int, int, int]:
        raise NotImplementedError

    def check_buffers(self, inputs, params, output, output_shape) -> None:
        """Buffers given as Buffer objects must hold the shapes the op will touch
        (input shapes, param_shapes, output shape); raw addresses are trusted."""
        shapes = [list(s) for _, s in inputs]
        expect = self.param_shapes(shapes, list(output_shape))
        pairs = [(b, s, "input") for b, s in inputs] + [(output, output_shape, "output")]
        pairs += [(b, s, f"param {n}") for b, s, n in zip(params, expect, self.param_names())]
        for buf, shape, what in pairs:
            if isinstance(buf, Buffer):
                _need(buf.numel >= _prod(shape),
                      f"{self.name}: {what} buffer holds {buf.numel} elements, needs {_prod(shape)}")

    def launch(self, inputs, params, output, output_shape, dtype, stream: Optional[Stream] = None):
        """Executor step: pack_args + grid, then run through teeny_dispatch."""
        self.check_buffers(inputs, params, output, output_shape)
        packer = DispatchPacker()
        self.pack_args(inputs, params, output, output_shape,
                       self.forward_output_row_stride(output_shape), packer)
        args, n = packer.array()
        cg = self.const_generics()
        cg_arr = (ctypes.c_int64 * max(1, len(cg)))(*cg)
        grid = (ctypes.c_uint32 * 3)(*self.grid(output_shape))
        check(lib.teeny_dispatch(self.entry_point_name().encode(), cg_arr, len(cg), args, n, grid,
                                 from_any(dtype).code, _h(stream)))


class _Elementwise(RuntimeOp):
    """relu.rs:119-180, gelu.rs:258-317, sigmoid.rs:389-448."""

    def __init__(self, block_size: int = 1024):
        self.block_size = int(block_size)

    def const_generics(self):
        return (self.block_size,)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        n = _prod(output_shape)
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(output)
        visitor.visit_i32(n)

    def grid(self, output_shape):
        n = _prod(output_shape)
        return (-(-n // self.block_size), 1, 1)

    # training hooks (core/teeny-core/src/model/mod.rs:213-280)
    def has_backward(self) -> bool:
        return True

    def backward_entry_point_name(self) -> str:
        return f"{self.backward_name}_entry_point"

    def pack_backward_args(self, inputs, params, output, output_shape, grad_output,
                           grad_output_row_stride, grad_inputs, grad_params, visitor):
        """(dy_ptr, saved, dx_ptr, n_elements): saved is the forward output for relu
        (relu.rs:156-172) and the forward input for gelu/silu (gelu.rs:293-309,
        sigmoid.rs:424-440)."""
        visitor.visit_ptr(grad_output)
        visitor.visit_ptr(output if self.saves_output else inputs[0][0])
        visitor.visit_ptr(grad_inputs[0])
        visitor.visit_i32(_prod(output_shape))

    def backward_grid(self, input_shapes, output_shape):
        return self.grid(output_shape)


class ReluForward(_Elementwise):
    name = "relu_forward"
    backward_name = "relu_backward"
    saves_output = True


class GeluForward(_Elementwise):
    name = "gelu_forward"
    backward_name = "gelu_backward"
    saves_output = False


class SiluForward(_Elementwise):
    name = "silu_forward"
    backward_name = "silu_backward"
    saves_output = False


class LayerNormForwardInferenceRuntimeOp(RuntimeOp):
    """layernorm.rs:486-561; BLOCK_N = 1024 and eps as the lowering passes them
    (kernels/teeny-kernels/src/graph/mod.rs:1184-1227)."""

    name = "layer_norm_forward_inference"

    def __init__(self, block_n: int = 1024, eps: float = 1e-5):
        self.block_n = int(block_n)
        self.eps = float(eps)

    def const_generics(self):
        return (self.block_n,)

    def param_shapes(self, input_shapes, output_shape):
        n = int(input_shapes[0][-1])
        return [[n], [n]]

    def param_names(self):
        return ("weight", "bias")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        shape = inputs[0][1]
        n = int(shape[-1])
        m = _prod(shape) // n
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(output)
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_i32(m)
        visitor.visit_i32(n)
        visitor.visit_f32(self.eps)

    def grid(self, output_shape):
        n = int(output_shape[-1])
        return (_prod(output_shape) // n, 1, 1)


class RmsNormForwardRuntimeOp(RuntimeOp):
    """A working RuntimeOp for rms_norm_forward (rmsnorm.rs:39-119); the
    reference's graph RuntimeOp for RMSNorm is a panicking stub
    (kernels/teeny-kernels/src/graph/mod.rs:454).  Params: weight [N] and the
    rrms output [M] (fp32), in the kernel's argument order."""

    name = "rms_norm_forward"

    def __init__(self, block_n: int = 1024, eps: float = 1e-8):
        self.block_n = int(block_n)
        self.eps = float(eps)

    def const_generics(self):
        return (self.block_n,)

    def param_shapes(self, input_shapes, output_shape):
        n = int(input_shapes[0][-1])
        m = _prod(input_shapes[0]) // n
        return [[n], [m]]

    def param_names(self):
        return ("weight", "rrms")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        shape = inputs[0][1]
        n = int(shape[-1])
        m = _prod(shape) // n
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(output)
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_i32(m)
        visitor.visit_i32(n)
        visitor.visit_f32(self.eps)

    def grid(self, output_shape):
        n = int(output_shape[-1])
        return (_prod(output_shape) // n, 1, 1)


POINTWISE_MEMBERS = {"relu": _lib.PW_RELU, "gelu": _lib.PW_GELU_TANH, "silu": _lib.PW_SILU,
                     "sigmoid": _lib.PW_SIGMOID, "tanh": _lib.PW_TANH}
Y_STYLE_MEMBERS = ("relu", "sigmoid", "tanh")


class PointwiseFuse(RuntimeOp):
    """The PointwiseFuse custom op's RuntimeOp (graph/optimizer/ops/
    pointwise_fuse.rs:155-268): params are the n-1 scratch buffers [n]
    (member outputs kept for backward), args (x, y, scratch..., n_elements),
    backward args (dy, y, dx, scratch..., n_elements) when every member has a
    y-style gradient; grid ceil(n / BLOCK_SIZE)."""

    def __init__(self, members, block_size: int = 1024):
        members = list(members)
        _need(2 <= len(members) <= 8, "PointwiseFuse: 2 to 8 members")
        for m in members:
            _need(m in POINTWISE_MEMBERS, f"PointwiseFuse: no fused kernel for member {m!r}")
        self.members = members
        self.block_size = int(block_size)
        self.name = "pointwise_fuse_" + "_".join(members)

    @property
    def n_scratch(self) -> int:
        return len(self.members) - 1

    def const_generics(self):
        return ()

    def param_shapes(self, input_shapes, output_shape):
        return [[_prod(output_shape)] for _ in range(self.n_scratch)]

    def param_names(self):
        return tuple(f"scratch{i}" for i in range(self.n_scratch))

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(output)
        for p in params[:self.n_scratch]:
            visitor.visit_ptr(p)
        visitor.visit_i32(_prod(output_shape))

    def grid(self, output_shape):
        return (-(-_prod(output_shape) // self.block_size), 1, 1)

    def has_backward(self) -> bool:
        return all(m in Y_STYLE_MEMBERS for m in self.members)

    def backward_entry_point_name(self) -> str:
        return f"{self.name}_backward_entry_point"

    def pack_backward_args(self, inputs, params, output, output_shape, grad_output, grad_output_row_stride,
                           grad_inputs, grad_params, visitor):
        visitor.visit_ptr(grad_output)
        visitor.visit_ptr(output)
        visitor.visit_ptr(grad_inputs[0])
        for p in params[:self.n_scratch]:
            visitor.visit_ptr(p)
        visitor.visit_i32(_prod(output_shape))

    def backward_grid(self, input_shapes, output_shape):
        return self.grid(output_shape)


class Conv2dForward(RuntimeOp):
    """conv2d.rs:523-618: const generics KH, KW, STRIDE_H, STRIDE_W, PAD_H,
    PAD_W, G, BLOCK_OW; args (x, w, y, B, C_IN, C_OUT, H, W, OH, OW)."""

    name = "conv2d_forward"
    has_bias = False

    def __init__(self, kh, kw, stride_h=1, stride_w=1, pad_h=0, pad_w=0, groups=1, block_ow=16):
        self.kh, self.kw = int(kh), int(kw)
        self.sh, self.sw = int(stride_h), int(stride_w)
        self.ph, self.pw = int(pad_h), int(pad_w)
        self.g = int(groups)
        self.block_ow = int(block_ow)

    def const_generics(self):
        return (self.kh, self.kw, self.sh, self.sw, self.ph, self.pw, self.g, self.block_ow)

    def output_hw(self, h, w):
        return ((h + 2 * self.ph - self.kh) // self.sh + 1, (w + 2 * self.pw - self.kw) // self.sw + 1)

    def param_shapes(self, input_shapes, output_shape):
        c_in, c_out = int(input_shapes[0][1]), int(output_shape[1])
        shapes = [[c_out, c_in // self.g, self.kh, self.kw]]
        if self.has_bias:
            shapes.append([c_out])
        return shapes

    def param_names(self):
        return ("weight", "bias") if self.has_bias else ("weight",)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        ish = inputs[0][1]
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        if self.has_bias:
            visitor.visit_ptr(params[1])
        visitor.visit_ptr(output)
        visitor.visit_i32(ish[0])
        visitor.visit_i32(ish[1])
        visitor.visit_i32(output_shape[1])
        visitor.visit_i32(ish[2])
        visitor.visit_i32(ish[3])
        visitor.visit_i32(output_shape[2])
        visitor.visit_i32(output_shape[3])

    def grid(self, output_shape):
        tiles = -(-int(output_shape[3]) // self.block_ow)
        return (int(output_shape[0]) * int(output_shape[1]) * int(output_shape[2]) * tiles, 1, 1)

    # training hooks (conv2d.rs:574-617): the combined conv2d_backward kernel
    def has_backward(self) -> bool:
        return True

    def backward_entry_point_name(self) -> str:
        return "conv2d_backward_entry_point"

    def pack_backward_args(self, inputs, params, output, output_shape, grad_output,
                           grad_output_row_stride, grad_inputs, grad_params, visitor):
        """(dy, x, w, dx, dw, B, C_IN, C_OUT, H, W, OH, OW), conv2d.rs:581-608."""
        ish = inputs[0][1]
        visitor.visit_ptr(grad_output)
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(grad_inputs[0])
        visitor.visit_ptr(grad_params[0])
        for v in (ish[0], ish[1], output_shape[1], ish[2], ish[3], output_shape[2], output_shape[3]):
            visitor.visit_i32(v)

    def backward_grid(self, input_shapes, output_shape):
        return self.grid(output_shape)


class Conv2dBnSiluForward(Conv2dForward):
    """conv2d_bn_silu.rs:200-245: params (weight, bn_scale, bn_shift); args
    (x, w, bn_scale, bn_shift, y, B, C_IN, C_OUT, H, W, OH, OW); the grid of
    conv2d_forward.  Inference only."""

    name = "conv2d_bn_silu_forward"

    def param_shapes(self, input_shapes, output_shape):
        c_in, c_out = int(input_shapes[0][1]), int(output_shape[1])
        return [[c_out, c_in // self.g, self.kh, self.kw], [c_out], [c_out]]

    def param_names(self):
        return ("weight", "bn_scale", "bn_shift")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        ish = inputs[0][1]
        visitor.visit_ptr(inputs[0][0])
        for p in params[:3]:
            visitor.visit_ptr(p)
        visitor.visit_ptr(output)
        for v in (ish[0], ish[1], output_shape[1], ish[2], ish[3], output_shape[2], output_shape[3]):
            visitor.visit_i32(v)

    def has_backward(self) -> bool:
        return False


class Conv2dBnSiluGemmForward(RuntimeOp):
    """conv2d_bn_silu_gemm.rs:200-260: 1x1 stride-1 conv as a GEMM; const
    generics BLOCK_M, BLOCK_N, BLOCK_K, GROUP_M; args (x, w, bn_scale,
    bn_shift, y, B, C_IN, C_OUT, M, y_row_stride) with each (b, c_out) row of
    y padded to a multiple of BLOCK_M."""

    name = "conv2d_bn_silu_gemm_forward"

    def __init__(self, block_m=32, block_n=32, block_k=32, group_m=8):
        self.block_m, self.block_n, self.block_k, self.group_m = int(block_m), int(block_n), int(block_k), int(group_m)

    def const_generics(self):
        return (self.block_m, self.block_n, self.block_k, self.group_m)

    def param_shapes(self, input_shapes, output_shape):
        return [[int(output_shape[1]), int(input_shapes[0][1])], [int(output_shape[1])], [int(output_shape[1])]]

    def param_names(self):
        return ("weight", "bn_scale", "bn_shift")

    def forward_output_row_elems(self, output_shape):
        return int(output_shape[2]) * int(output_shape[3])

    def forward_output_row_stride(self, output_shape):
        m = self.forward_output_row_elems(output_shape)
        return -(-m // self.block_m) * self.block_m

    def check_buffers(self, inputs, params, output, output_shape):
        rows = int(output_shape[0]) * int(output_shape[1])
        RuntimeOp.check_buffers(self, inputs, params, None, output_shape)
        if isinstance(output, Buffer):
            _need(output.numel >= rows * self.forward_output_row_stride(output_shape),
                  f"{self.name}: y must hold the padded rows")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        ish = inputs[0][1]
        visitor.visit_ptr(inputs[0][0])
        for p in params[:3]:
            visitor.visit_ptr(p)
        visitor.visit_ptr(output)
        for v in (ish[0], ish[1], output_shape[1], int(output_shape[2]) * int(output_shape[3]), output_row_stride):
            visitor.visit_i32(v)

    def grid(self, output_shape):
        m = int(output_shape[2]) * int(output_shape[3])
        return (int(output_shape[0]) * -(-m // self.block_m) * -(-int(output_shape[1]) // self.block_n), 1, 1)

    def has_backward(self) -> bool:
        return False


class Conv2dBnSiluTiledForward(RuntimeOp):
    """conv2d_bn_silu_tiled.rs:214-293: const generics KH, KW, STRIDE_H,
    STRIDE_W, PAD_H, PAD_W, BLOCK_OW, BLOCK_N (groups 1); args (x, w,
    bn_scale, bn_shift, y, B, C_IN, C_OUT, H, W, OH, OW, y_col_stride), each
    oh row of y padded to a multiple of BLOCK_OW."""

    name = "conv2d_bn_silu_tiled_forward"

    def __init__(self, kh, kw, stride_h=1, stride_w=1, pad_h=0, pad_w=0, block_ow=16, block_n=16):
        self.kh, self.kw, self.sh, self.sw = int(kh), int(kw), int(stride_h), int(stride_w)
        self.ph, self.pw, self.block_ow, self.block_n = int(pad_h), int(pad_w), int(block_ow), int(block_n)

    def const_generics(self):
        return (self.kh, self.kw, self.sh, self.sw, self.ph, self.pw, self.block_ow, self.block_n)

    def param_shapes(self, input_shapes, output_shape):
        c_in, c_out = int(input_shapes[0][1]), int(output_shape[1])
        return [[c_out, c_in, self.kh, self.kw], [c_out], [c_out]]

    def param_names(self):
        return ("weight", "bn_scale", "bn_shift")

    def forward_output_row_stride(self, output_shape):
        return -(-int(output_shape[3]) // self.block_ow) * self.block_ow

    def check_buffers(self, inputs, params, output, output_shape):
        RuntimeOp.check_buffers(self, inputs, params, None, output_shape)
        if isinstance(output, Buffer):
            rows = int(output_shape[0]) * int(output_shape[1]) * int(output_shape[2])
            _need(output.numel >= rows * self.forward_output_row_stride(output_shape),
                  f"{self.name}: y must hold the padded rows")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        ish = inputs[0][1]
        visitor.visit_ptr(inputs[0][0])
        for p in params[:3]:
            visitor.visit_ptr(p)
        visitor.visit_ptr(output)
        for v in (ish[0], ish[1], output_shape[1], ish[2], ish[3], output_shape[2], output_shape[3],
                  output_row_stride):
            visitor.visit_i32(v)

    def grid(self, output_shape):
        tiles_ow = -(-int(output_shape[3]) // self.block_ow)
        tiles_n = -(-int(output_shape[1]) // self.block_n)
        return (int(output_shape[0]) * int(output_shape[2]) * tiles_n * tiles_ow, 1, 1)

    def has_backward(self) -> bool:
        return False


class Conv2dBiasForward(Conv2dForward):
    """conv2d.rs:766-820: the conv2d_forward contract plus bias after w."""

    name = "conv2d_bias_forward"
    has_bias = True


class FlashAttention2Forward(RuntimeOp):
    """flash_attn2.rs:52-158.  The reference has no RuntimeOp for it (its
    tests launch it directly, tests/test_flash_attn2.rs:96-180); this mirrors
    that launch: args (q, k, v, o, l, n_ctx_q, n_ctx_k, softmax_scale,
    neg_inf), const HEAD_DIM, grid (N_CTX_Q, BH, 1).  Inputs are q, k, v of
    shape [BH, N, HEAD_DIM]; params[0] is the l (logsumexp) buffer."""

    name = "flash_attention2_forward"

    def __init__(self, head_dim: int, softmax_scale: Optional[float] = None, causal: bool = False):
        self.head_dim = int(head_dim)
        self.softmax_scale = float(softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(head_dim))
        self.causal = bool(causal)

    def const_generics(self):
        # the reference kernel has HEAD_DIM only; CAUSAL is this library's extension
        return (self.head_dim, 1) if self.causal else (self.head_dim,)

    def n_activation_inputs(self):
        return 3

    def param_shapes(self, input_shapes, output_shape):
        return [[int(output_shape[0]), int(output_shape[1])]]

    def param_names(self):
        return ("l",)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(inputs[1][0])
        visitor.visit_ptr(inputs[2][0])
        visitor.visit_ptr(output)
        visitor.visit_ptr(params[0])
        visitor.visit_i32(inputs[0][1][1])
        visitor.visit_i32(inputs[1][1][1])
        visitor.visit_f32(self.softmax_scale)
        visitor.visit_f32(float("-inf"))

    def grid(self, output_shape):
        return (int(output_shape[1]), int(output_shape[0]), 1)


class MultiHeadAttentionRuntimeOp(FlashAttention2Forward):
    """Lowering of Op::MultiHeadAttention{q_num_heads, kv_num_heads}
    (core/teeny-core/src/graph/mod.rs:1240-1246) — a TODO arm of the
    reference's lowering (kernels/teeny-kernels/src/graph/mod.rs:2477-2481) —
    onto the flash kernel, with grouped K/V heads.  Inputs q [B*Q_HEADS, Nq,
    HEAD_DIM], k and v [B*KV_HEADS, Nk, HEAD_DIM]; params[0] is l; the packed
    arguments are flash_attention2_forward's; const generics HEAD_DIM, CAUSAL,
    Q_HEADS, KV_HEADS; grid (Nq, B*Q_HEADS, 1)."""

    name = "multi_head_attention_forward"

    def __init__(self, q_num_heads: int, kv_num_heads: int, head_dim: int, causal: bool = False,
                 softmax_scale: Optional[float] = None):
        super().__init__(head_dim, softmax_scale, causal)
        _need(q_num_heads > 0 and kv_num_heads > 0 and q_num_heads % kv_num_heads == 0,
              "multi_head_attention: q_num_heads must be a positive multiple of kv_num_heads")
        self.q_num_heads, self.kv_num_heads = int(q_num_heads), int(kv_num_heads)

    def const_generics(self):
        return (self.head_dim, int(self.causal), self.q_num_heads, self.kv_num_heads)


class W8A16LinearRuntimeOp(RuntimeOp):
    """Lowering of Op::QLinearMatMul / Op::MatMulInteger with teeny-quant
    per-output-channel int8 weights — TODO arms of the reference's lowering
    (kernels/teeny-kernels/src/graph/mod.rs:2595-2601) — as linear_forward
    (nn/mlp/linear.rs:20-116) on dequantize_affine's weights
    (utilities/teeny-quant/src/quant/affine.rs:151-161).  Input x bf16 [M, K];
    params qweight int8 [N, K], scale fp32 [N] (and bias fp32 [N]); const
    generics USE_BIAS, ACT; args (x, qweight, scale, bias, y, M, N, K)."""

    name = "w8a16_linear_forward"

    def __init__(self, use_bias: bool = False, act: Optional[str] = None):
        self.use_bias = bool(use_bias)
        self.act = ACTS[act]

    def const_generics(self):
        return (int(self.use_bias), self.act)

    def param_shapes(self, input_shapes, output_shape):
        k, n = int(input_shapes[0][1]), int(output_shape[1])
        return [[n, k], [n], [n]] if self.use_bias else [[n, k], [n]]

    def param_names(self):
        return ("qweight", "scale", "bias") if self.use_bias else ("qweight", "scale")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        m, n = int(output_shape[0]), int(output_shape[1])
        k = int(inputs[0][1][1])
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_ptr(params[2] if self.use_bias else None)
        visitor.visit_ptr(output)
        for v in (m, n, k):
            visitor.visit_i32(v)

    def grid(self, output_shape):
        return (-(-int(output_shape[0]) // 256) * -(-int(output_shape[1]) // 256), 1, 1)


class W8A16Conv2dRuntimeOp(RuntimeOp):
    """Lowering of Op::QLinearConv / Op::ConvInteger with teeny-quant int8
    weights (TODO arms, kernels/teeny-kernels/src/graph/mod.rs:2595-2601):
    conv2d_bias_forward (nn/conv/conv2d.rs:642-764) on dequantized weights,
    NHWC.  Input x bf16 [B, H, W, C_IN]; params qweight int8 [C_OUT, KH, KW,
    C_IN/G], scale fp32 [C_OUT] (and bias fp32 [C_OUT]); output [B, OH, OW,
    C_OUT]; const generics KH..BLOCK_OW of conv2d_forward plus USE_BIAS, ACT;
    args (x, qweight, scale, bias, y, B, C_IN, C_OUT, H, W, OH, OW)."""

    name = "w8a16_conv2d_forward"

    def __init__(self, kh, kw, stride_h=1, stride_w=1, pad_h=0, pad_w=0, groups=1, block_ow=16,
                 use_bias=False, act: Optional[str] = None):
        self.conv = Conv2dForward(kh, kw, stride_h, stride_w, pad_h, pad_w, groups, block_ow)
        self.use_bias = bool(use_bias)
        self.act = ACTS[act]

    def const_generics(self):
        return self.conv.const_generics() + (int(self.use_bias), self.act)

    def param_shapes(self, input_shapes, output_shape):
        c = self.conv
        cin, cout = int(input_shapes[0][3]), int(output_shape[3])
        shapes = [[cout, c.kh, c.kw, cin // c.g], [cout]]
        return shapes + [[cout]] if self.use_bias else shapes

    def param_names(self):
        return ("qweight", "scale", "bias") if self.use_bias else ("qweight", "scale")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        ish = inputs[0][1]
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_ptr(params[2] if self.use_bias else None)
        visitor.visit_ptr(output)
        for v in (ish[0], ish[3], output_shape[3], ish[1], ish[2], output_shape[1], output_shape[2]):
            visitor.visit_i32(v)

    def grid(self, output_shape):
        b, oh, ow, cout = (int(v) for v in output_shape)
        return (b * cout * oh * -(-ow // self.conv.block_ow), 1, 1)


class QuantizeAffineRuntimeOp(RuntimeOp):
    """Lowering of Op::QuantizeLinear{axis} (TODO arm, kernels/teeny-kernels/
    src/graph/mod.rs:2691-2697) to teeny-quant's quantize_affine
    (utilities/teeny-quant/src/quant/affine.rs:55-148).  Input fp32 data of
    any shape; output int8 q of that shape; params scales fp32 [groups] and
    zero_points int32 [groups]; const generics GRANULARITY, AXIS, GROUP_SIZE,
    SYMMETRIC, BITS; args (data, q, scales, zero_points, groups = null, ndim,
    dims as i64)."""

    name = "quantize_affine"

    def __init__(self, granularity="channel", axis=0, group_size=1, symmetric=True, bits=8):
        self.gran = GRANULARITY[granularity] if isinstance(granularity, str) else int(granularity)
        self.granularity = granularity
        self.axis, self.group_size = int(axis), int(group_size)
        self.symmetric, self.bits = bool(symmetric), int(bits)

    def const_generics(self):
        return (self.gran, self.axis, self.group_size, int(self.symmetric), self.bits)

    def param_shapes(self, input_shapes, output_shape):
        ng = quant_num_groups(list(input_shapes[0]), self.granularity, self.axis, self.group_size)
        return [[max(ng, 1)], [max(ng, 1)]]

    def param_names(self):
        return ("scales", "zero_points")

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        shape = list(inputs[0][1])
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(output)
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_ptr(None)
        visitor.visit_i32(len(shape))
        for d in shape:
            visitor.visit_i64(d)

    def grid(self, output_shape):
        return (-(-_prod(output_shape) // 256), 1, 1)


class DequantizeAffineRuntimeOp(QuantizeAffineRuntimeOp):
    """Lowering of Op::DequantizeLinear{axis} (TODO arm, graph/mod.rs:2691-2697)
    to dequantize_affine (affine.rs:151-161).  Input int8 q; output fp32 of the
    same shape; params scales fp32 [groups] and zero_points int32 [groups];
    const generics GRANULARITY, AXIS, GROUP_SIZE; args (q, scales,
    zero_points, out, ndim, dims as i64)."""

    name = "dequantize_affine"

    def const_generics(self):
        return (self.gran, self.axis, self.group_size)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        shape = list(inputs[0][1])
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1])
        visitor.visit_ptr(output)
        visitor.visit_i32(len(shape))
        for d in shape:
            visitor.visit_i64(d)


class LinearForward(RuntimeOp):
    """linear.rs:250-320: const generics USE_BIAS, BLOCK_M, BLOCK_N, BLOCK_K,
    GROUP_M; args (x, w, b, y, M, N, K, stride_xm, stride_xk, stride_wn,
    stride_wk, stride_ym, stride_yn); b is null without bias."""

    name = "linear_forward"

    def __init__(self, use_bias=True, block_m=64, block_n=64, block_k=32, group_m=8):
        self.use_bias = bool(use_bias)
        self.block_m, self.block_n, self.block_k, self.group_m = block_m, block_n, block_k, group_m

    def const_generics(self):
        return (int(self.use_bias), self.block_m, self.block_n, self.block_k, self.group_m)

    def param_shapes(self, input_shapes, output_shape):
        k, n = int(input_shapes[0][1]), int(output_shape[1])
        return [[n, k], [n]] if self.use_bias else [[n, k]]

    def param_names(self):
        return ("weight", "bias") if self.use_bias else ("weight",)

    def pack_args(self, inputs, params, output, output_shape, output_row_stride, visitor):
        m, n = int(output_shape[0]), int(output_shape[1])
        k = int(inputs[0][1][1])
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(params[1] if self.use_bias else None)
        visitor.visit_ptr(output)
        for v in (m, n, k, k, 1, k, 1, output_row_stride, 1):
            visitor.visit_i32(v)

    def grid(self, output_shape):
        pm = -(-int(output_shape[0]) // self.block_m)
        pn = -(-int(output_shape[1]) // self.block_n)
        return (pm * pn, 1, 1)

    # training hooks (linear.rs:322-385): linear_backward
    def has_backward(self) -> bool:
        return True

    def backward_entry_point_name(self) -> str:
        return "linear_backward_entry_point"

    def backward_grad_output_row_stride(self, output_shape, elem_bytes=4) -> int:
        """dy rows padded to 16 bytes (linear.rs:329-334)."""
        n = int(output_shape[-1])
        align = 16 // elem_bytes
        return -(-n // align) * align

    def pack_backward_args(self, inputs, params, output, output_shape, grad_output,
                           grad_output_row_stride, grad_inputs, grad_params, visitor):
        """(x, w, dy, dx, dw, db, M, N, K, stride_xm, stride_xk, stride_wk,
        stride_wn, stride_dym, stride_dyn, stride_dxm, stride_dxk, stride_dwk,
        stride_dwn, stride_dbn), linear.rs:341-384; db is null without bias."""
        m, n = int(output_shape[0]), int(output_shape[1])
        k = int(inputs[0][1][1])
        visitor.visit_ptr(inputs[0][0])
        visitor.visit_ptr(params[0])
        visitor.visit_ptr(grad_output)
        visitor.visit_ptr(grad_inputs[0])
        visitor.visit_ptr(grad_params[0])
        visitor.visit_ptr(grad_params[1] if self.use_bias else None)
        for v in (m, n, k, k, 1, 1, k, grad_output_row_stride, 1, k, 1, 1, k, 1):
            visitor.visit_i32(v)

    def backward_grid(self, input_shapes, output_shape):
        pm = -(-int(output_shape[0]) // self.block_m)
        pn = -(-int(output_shape[1]) // self.block_n)
        pk = -(-int(input_shapes[0][1]) // self.block_k)
        return (pm * pn * pk, 1, 1)


# ── direct entry points on Buffers ──────────────────────────────────────────


def _out(like: Buffer, out: Optional[Buffer], shape=None, dtype=None) -> Buffer:
    """The output buffer: `out` if given (its size and dtype must match), else a new one."""
    shape = tuple(shape if shape is not None else like.shape)
    dtype = from_any(dtype or like.dtype)
    if out is not None:
        _need(out.numel == _prod(shape), f"output holds {out.numel} elements, op writes {_prod(shape)}")
        _need(out.dtype == dtype, f"output dtype {out.dtype.name}, op writes {dtype.name}")
        return out
    return Buffer(dtype, shape)


# Shape rules of each entry point, as pure functions of buffer shapes (so the
# rules are testable without a device).  Every wrapper below checks its
# buffers with these before calling the C ABI, which cannot see allocation
# sizes through raw pointers.

def linear_dims(x_shape, w_shape, b_shape=None) -> Tuple[int, int, int]:
    _need(len(x_shape) == 2 and len(w_shape) == 2, "linear: x and w must be 2-D")
    m, k = x_shape
    n, kw = w_shape
    _need(k == kw, f"linear: x has K={k}, w has K={kw}")
    _need(b_shape is None or _prod(b_shape) == n, f"linear: bias must have {n} elements")
    return int(m), int(n), int(k)


def w8a16_dims(x_shape, q_shape, scale_shape, bias_shape=None) -> Tuple[int, int, int]:
    m, n, k = linear_dims(x_shape, q_shape, bias_shape)
    _need(_prod(scale_shape) == n, f"w8a16: scale must have N={n} elements, has {_prod(scale_shape)}")
    return m, n, k


def conv2d_dims(x_shape, w_shape, stride, padding, groups, layout, b_shape=None):
    """-> (B, Cin, Cout, H, W, OH, OW, KH, KW, sh, sw, ph, pw) with the reference's shape rules."""
    sh, sw = (stride, stride) if isinstance(stride, int) else stride
    ph, pw = (padding, padding) if isinstance(padding, int) else padding
    _need(len(x_shape) == 4 and len(w_shape) == 4, "conv2d: x and w must be 4-D")
    if layout == "nhwc":
        b, h, wd, cin = x_shape
        cout, kh, kw, cg = w_shape
    else:
        b, cin, h, wd = x_shape
        cout, cg, kh, kw = w_shape
    _need(groups > 0 and cin % groups == 0 and cout % groups == 0,
          f"conv2d: groups={groups} must divide C_IN={cin} and C_OUT={cout}")
    _need(cg == cin // groups, f"conv2d: weight has {cg} input channels per group, expected {cin // groups}")
    _need(b_shape is None or _prod(b_shape) == cout, f"conv2d: bias must have {cout} elements")
    _need(h + 2 * ph >= kh and wd + 2 * pw >= kw, "conv2d: kernel larger than padded input")
    oh, ow = (h + 2 * ph - kh) // sh + 1, (wd + 2 * pw - kw) // sw + 1
    return b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw


def attention_dims(q_shape, k_shape, v_shape, lse_shape=None):
    _need(len(q_shape) == 3 and len(k_shape) == 3 and len(v_shape) == 3,
          "attention: q, k, v must be [BH, N, D]")
    bh, nq, d = q_shape
    _need(tuple(k_shape) == tuple(v_shape), "attention: k and v shapes differ")
    _need(k_shape[0] == bh and k_shape[2] == d, "attention: k/v must share BH and D with q")
    _need(lse_shape is None or _prod(lse_shape) == bh * nq, f"attention: lse must have {bh * nq} elements")
    return int(bh), int(nq), int(k_shape[1]), int(d)


def norm_dims(x_shape, weight_shape, bias_shape=None, rrms_shape=None):
    n = int(x_shape[-1])
    m = _prod(x_shape) // n
    _need(_prod(weight_shape) == n, f"norm: weight must have N={n} elements")
    _need(bias_shape is None or _prod(bias_shape) == n, f"norm: bias must have N={n} elements")
    _need(rrms_shape is None or _prod(rrms_shape) == m, f"norm: rrms must have M={m} elements")
    return m, n


def relu(x: Buffer, y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    y = _out(x, y)
    check(lib.teeny_relu_forward(x.ptr, y.ptr, x.numel, x.dtype.code, _h(stream)))
    return y


def gelu(x: Buffer, y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    y = _out(x, y)
    check(lib.teeny_gelu_forward(x.ptr, y.ptr, x.numel, x.dtype.code, _h(stream)))
    return y


def silu(x: Buffer, y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    y = _out(x, y)
    check(lib.teeny_silu_forward(x.ptr, y.ptr, x.numel, x.dtype.code, _h(stream)))
    return y


def _act_grad(fn, what: str, dy: Buffer, saved: Buffer, dx: Optional[Buffer],
              stream: Optional[Stream]) -> Buffer:
    _need(dy.dtype == saved.dtype and dy.numel == saved.numel,
          f"{what}: dy and the saved tensor must match in dtype and size")
    dx = _out(dy, dx)
    check(fn(dy.ptr, saved.ptr, dx.ptr, dy.numel, dy.dtype.code, _h(stream)))
    return dx


def relu_backward(dy: Buffer, y: Buffer, dx: Optional[Buffer] = None,
                  stream: Optional[Stream] = None) -> Buffer:
    """relu.rs:67-117: dx = dy where the forward OUTPUT y > 0, else 0."""
    return _act_grad(lib.teeny_relu_backward, "relu_backward", dy, y, dx, stream)


def gelu_backward(dy: Buffer, x: Buffer, dx: Optional[Buffer] = None,
                  stream: Optional[Stream] = None) -> Buffer:
    """gelu.rs:81-139: dy times the tanh-GELU derivative at the forward input x."""
    return _act_grad(lib.teeny_gelu_backward, "gelu_backward", dy, x, dx, stream)


def silu_backward(dy: Buffer, x: Buffer, dx: Optional[Buffer] = None,
                  stream: Optional[Stream] = None) -> Buffer:
    """sigmoid.rs:161-210: dy * (s + y - y s), s = sigmoid(x), y = x s."""
    return _act_grad(lib.teeny_silu_backward, "silu_backward", dy, x, dx, stream)


def layer_norm(x: Buffer, weight: Buffer, bias: Buffer, eps: float = 1e-5,
               y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    m, n = norm_dims(x.shape, weight.shape, bias.shape)
    _need(weight.dtype == x.dtype and bias.dtype == x.dtype, "layer_norm: weight/bias dtype must match x")
    y = _out(x, y)
    check(lib.teeny_layer_norm_forward_inference(x.ptr, y.ptr, weight.ptr, bias.ptr, m, n, eps,
                                                 x.dtype.code, _h(stream)))
    return y


def rms_norm(x: Buffer, weight: Buffer, eps: float = 1e-8, y: Optional[Buffer] = None,
             rrms: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    m, n = norm_dims(x.shape, weight.shape, None, rrms.shape if rrms is not None else None)
    _need(weight.dtype == x.dtype, "rms_norm: weight dtype must match x")
    _need(rrms is None or rrms.dtype == f32, "rms_norm: rrms is fp32")
    y = _out(x, y)
    check(lib.teeny_rms_norm_forward(x.ptr, y.ptr, weight.ptr, rrms.ptr if rrms is not None else None,
                                     m, n, eps, x.dtype.code, _h(stream)))
    return y


def layer_norm_train(x: Buffer, weight: Buffer, bias: Buffer, eps: float = 1e-5, y: Optional[Buffer] = None,
                     mean: Optional[Buffer] = None, rstd: Optional[Buffer] = None,
                     stream: Optional[Stream] = None):
    """layernorm.rs:162-298: (y, mean fp32 [M], rstd fp32 [M])."""
    m, n = norm_dims(x.shape, weight.shape, bias.shape)
    y = _out(x, y)
    mean = _out(x, mean, (m,), f32)
    rstd = _out(x, rstd, (m,), f32)
    check(lib.teeny_layer_norm_forward(x.ptr, y.ptr, weight.ptr, bias.ptr, mean.ptr, rstd.ptr, m, n, eps,
                                       x.dtype.code, _h(stream)))
    return y, mean, rstd


def layer_norm_backward(dy: Buffer, x: Buffer, weight: Buffer, mean: Buffer, rstd: Buffer,
                        dweight: Optional[Buffer] = None, dbias: Optional[Buffer] = None,
                        dx: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """layernorm.rs:300-482: returns dx; dweight / dbias (fp32 [N]) accumulate in place."""
    m, n = norm_dims(x.shape, weight.shape)
    _need(dy.shape == x.shape and dy.dtype == x.dtype and weight.dtype == x.dtype, "layer_norm_backward: dy/x/weight")
    _need(mean.numel == m and rstd.numel == m and mean.dtype == f32 and rstd.dtype == f32,
          f"layer_norm_backward: mean/rstd fp32 [{m}]")
    for g in (dweight, dbias):
        _need(g is None or (g.numel == n and g.dtype == f32), f"layer_norm_backward: dweight/dbias fp32 [{n}]")
    dx = _out(x, dx)
    check(lib.teeny_layer_norm_backward(dy.ptr, x.ptr, dx.ptr, weight.ptr, dweight.ptr if dweight else None,
                                        dbias.ptr if dbias else None, mean.ptr, rstd.ptr, m, n, x.dtype.code,
                                        _h(stream)))
    return dx


def rms_norm_backward(dy: Buffer, x: Buffer, weight: Buffer, rrms: Buffer, dweight: Optional[Buffer] = None,
                      dx: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """rmsnorm.rs:135-277: returns dx; dweight (fp32 [N]) accumulates in place."""
    m, n = norm_dims(x.shape, weight.shape, None, rrms.shape)
    _need(dy.shape == x.shape and dy.dtype == x.dtype and weight.dtype == x.dtype, "rms_norm_backward: dy/x/weight")
    _need(rrms.dtype == f32 and (dweight is None or (dweight.numel == n and dweight.dtype == f32)),
          "rms_norm_backward: rrms / dweight fp32")
    dx = _out(x, dx)
    check(lib.teeny_rms_norm_backward(dy.ptr, x.ptr, dx.ptr, weight.ptr, dweight.ptr if dweight else None, rrms.ptr,
                                      m, n, x.dtype.code, _h(stream)))
    return dx


def norm_backward_workspace_size(m: int, n: int, rms: bool, dtype=bf16) -> int:
    out = ctypes.c_size_t(0)
    check(lib.teeny_norm_backward_workspace_size(m, n, int(bool(rms)), from_any(dtype).code, ctypes.byref(out)))
    return int(out.value)


ACTS = {None: _lib.ACT_NONE, "none": _lib.ACT_NONE, "relu": _lib.ACT_RELU,
        "gelu": _lib.ACT_GELU_TANH, "gelu_tanh": _lib.ACT_GELU_TANH, "silu": _lib.ACT_SILU}


def norm_act(x: Buffer, weight: Buffer, bias: Optional[Buffer], eps: float, rms: bool, act: str,
             y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    m, n = norm_dims(x.shape, weight.shape, bias.shape if bias is not None else None)
    _need(rms or bias is not None, "norm_act: LayerNorm needs a bias")
    y = _out(x, y)
    check(lib.teeny_norm_act_forward(x.ptr, y.ptr, weight.ptr, bias.ptr if bias is not None else None,
                                     m, n, eps, int(rms), ACTS[act], x.dtype.code, _h(stream)))
    return y


def conv2d(x: Buffer, w: Buffer, bias: Optional[Buffer] = None, stride=(1, 1), padding=(0, 0),
           groups: int = 1, act: Optional[str] = None, layout: str = "nchw",
           y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """x NCHW [B,C,H,W] or NHWC [B,H,W,C]; w [Cout,Cin/G,KH,KW] (NCHW) or
    [Cout,KH,KW,Cin/G] (NHWC)."""
    nhwc = layout.lower() == "nhwc"
    b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw = conv2d_dims(
        x.shape, w.shape, stride, padding, groups, "nhwc" if nhwc else "nchw",
        bias.shape if bias is not None else None)
    _need(w.dtype == x.dtype and (bias is None or bias.dtype == x.dtype),
          "conv2d: w/bias dtype must match x")
    yshape = (b, oh, ow, cout) if nhwc else (b, cout, oh, ow)
    y = _out(x, y, yshape)
    prm = _lib.Conv2dParams(kh, kw, sh, sw, ph, pw, groups, ACTS[act])
    lay = _lib.NHWC if nhwc else _lib.NCHW
    if bias is None:
        check(lib.teeny_conv2d_forward(x.ptr, w.ptr, y.ptr, b, cin, cout, h, wd, oh, ow,
                                       ctypes.byref(prm), x.dtype.code, lay, _h(stream)))
    else:
        check(lib.teeny_conv2d_bias_forward(x.ptr, w.ptr, bias.ptr, y.ptr, b, cin, cout, h, wd, oh,
                                            ow, ctypes.byref(prm), x.dtype.code, lay, _h(stream)))
    return y


def _chain_args(members, scratch):
    ops = (ctypes.c_int32 * len(members))(*(POINTWISE_MEMBERS[m] for m in members))
    sc = None
    if scratch is not None:
        _need(len(scratch) >= len(members) - 1, "pointwise chain: one scratch buffer per member but the last")
        sc = (ctypes.c_void_p * max(1, len(scratch)))(*((b.ptr if b is not None else None) for b in scratch))
    return ops, sc


def pointwise_chain(x: Buffer, members, y: Optional[Buffer] = None, scratch=None,
                    stream: Optional[Stream] = None) -> Buffer:
    """PointwiseFuse forward (pointwise_fuse.rs:73-233): the members applied in
    one pass; scratch[i] (optional) receives member i's output."""
    y = _out(x, y)
    for b in scratch or []:
        _need(b is None or (b.numel == x.numel and b.dtype == x.dtype), "pointwise chain: scratch like x")
    ops, sc = _chain_args(members, scratch)
    check(lib.teeny_pointwise_chain_forward(x.ptr, y.ptr, sc, ops, len(members), x.numel, x.dtype.code, _h(stream)))
    return y


def pointwise_chain_backward(dy: Buffer, y: Buffer, scratch, members, dx: Optional[Buffer] = None,
                             stream: Optional[Stream] = None) -> Buffer:
    """The fused chain's backward (members relu / sigmoid / tanh): dx from dy,
    the chain output y and the kept member outputs."""
    _need(dy.numel == y.numel and dy.dtype == y.dtype, "pointwise chain backward: dy like y")
    for b in scratch:
        _need(b.numel == y.numel and b.dtype == y.dtype, "pointwise chain backward: scratch like y")
    dx = _out(dy, dx)
    ops, sc = _chain_args(members, scratch)
    check(lib.teeny_pointwise_chain_backward(dy.ptr, y.ptr, dx.ptr, sc, ops, len(members), dy.numel, dy.dtype.code,
                                             _h(stream)))
    return dx


def conv2d_bn_act(x: Buffer, w: Buffer, bn_scale: Buffer, bn_shift: Buffer, stride=(1, 1), padding=(0, 0),
                  groups: int = 1, act: Optional[str] = "silu", layout: str = "nchw", y: Optional[Buffer] = None,
                  y_strides=None, stream: Optional[Stream] = None) -> Buffer:
    """conv2d_bn_silu.rs:26-199 with any activation: act(bn_scale[c] * conv + bn_shift[c]),
    bn_scale / bn_shift fp32 [C_OUT] (BatchNorm folded by the caller).  y_strides (NCHW)
    addresses padded output rows; y must then hold the strided extent."""
    nhwc = layout.lower() == "nhwc"
    b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw = conv2d_dims(
        x.shape, w.shape, stride, padding, groups, "nhwc" if nhwc else "nchw")
    _need(w.dtype == x.dtype, "conv2d_bn_act: w dtype must match x")
    _need(bn_scale.numel == cout and bn_shift.numel == cout and bn_scale.dtype == f32 and bn_shift.dtype == f32,
          f"conv2d_bn_act: bn_scale / bn_shift fp32 [{cout}]")
    yshape = (b, oh, ow, cout) if nhwc else (b, cout, oh, ow)
    strides = None
    if y_strides is not None:
        _need(y is not None and not nhwc, "conv2d_bn_act: y_strides needs an NCHW y buffer")
        strides = (ctypes.c_int64 * 4)(*y_strides)
        _need(y.numel >= (b - 1) * y_strides[0] + (cout - 1) * y_strides[1] + (oh - 1) * y_strides[2] + ow,
              "conv2d_bn_act: y smaller than its strided extent")
    else:
        y = _out(x, y, yshape)
    prm = _lib.Conv2dParams(kh, kw, sh, sw, ph, pw, groups, ACTS[act])
    check(lib.teeny_conv2d_bn_act_forward(x.ptr, w.ptr, bn_scale.ptr, bn_shift.ptr, y.ptr, b, cin, cout, h, wd, oh,
                                          ow, strides, ctypes.byref(prm), x.dtype.code,
                                          _lib.NHWC if nhwc else _lib.NCHW, _h(stream)))
    return y


def fold_batchnorm(gamma, beta, mean, var, eps=1e-5):
    """Host-side BatchNorm folding, the convention of conv2d_bn_silu.rs:32-35:
    bn_scale = gamma / sqrt(var + eps), bn_shift = beta - bn_scale * mean (fp32)."""
    gamma, beta, mean, var = (np.asarray(a, np.float32) for a in (gamma, beta, mean, var))
    scale = (gamma / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return scale, (beta - scale * mean).astype(np.float32)


def _conv_bwd_args(x_shape, w_shape, stride, padding, groups, layout, dtype):
    nhwc = layout.lower() == "nhwc"
    geo = conv2d_dims(x_shape, w_shape, stride, padding, groups, "nhwc" if nhwc else "nchw")
    b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw = geo
    prm = _lib.Conv2dParams(kh, kw, sh, sw, ph, pw, groups, 0)
    yshape = (b, oh, ow, cout) if nhwc else (b, cout, oh, ow)
    return (b, cin, cout, h, wd, oh, ow), prm, _lib.NHWC if nhwc else _lib.NCHW, yshape


def conv2d_backward_dx(dy: Buffer, w: Buffer, x_shape, stride=(1, 1), padding=(0, 0), groups: int = 1,
                       layout: str = "nchw", dx: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """conv2d.rs:171-284: dx of x's shape from dy (y's shape) and w."""
    dims, prm, lay, yshape = _conv_bwd_args(x_shape, w.shape, stride, padding, groups, layout, dy.dtype)
    _need(tuple(dy.shape) == tuple(yshape) and w.dtype == dy.dtype, f"conv2d_backward_dx: dy must be {yshape}")
    dx = _out(dy, dx, tuple(x_shape))
    check(lib.teeny_conv2d_backward_dx(dy.ptr, w.ptr, dx.ptr, *dims, ctypes.byref(prm), dy.dtype.code, lay,
                                       _h(stream)))
    return dx


def conv2d_backward_dw(dy: Buffer, x: Buffer, w_shape, stride=(1, 1), padding=(0, 0), groups: int = 1,
                       layout: str = "nchw", dw: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """conv2d.rs:286-397: dw of w's shape from dy and x."""
    dims, prm, lay, yshape = _conv_bwd_args(x.shape, w_shape, stride, padding, groups, layout, dy.dtype)
    _need(tuple(dy.shape) == tuple(yshape) and x.dtype == dy.dtype, f"conv2d_backward_dw: dy must be {yshape}")
    dw = _out(dy, dw, tuple(w_shape))
    check(lib.teeny_conv2d_backward_dw(dy.ptr, x.ptr, dw.ptr, *dims, ctypes.byref(prm), dy.dtype.code, lay,
                                       _h(stream)))
    return dw


def conv2d_backward_workspace_size(x_shape, w_shape, stride=(1, 1), padding=(0, 0), groups: int = 1,
                                   dtype=bf16, layout: str = "nhwc") -> int:
    dims, prm, lay, _ = _conv_bwd_args(x_shape, w_shape, stride, padding, groups, layout, dtype)
    out = ctypes.c_size_t(0)
    check(lib.teeny_conv2d_backward_workspace_size(*dims, ctypes.byref(prm), from_any(dtype).code, lay,
                                                   ctypes.byref(out)))
    return int(out.value)


def conv2d_workspace_size(x_shape, w_shape, stride=(1, 1), padding=(0, 0), groups: int = 1,
                          dtype=bf16, layout: str = "nhwc") -> int:
    """Stream workspace bytes that let this conv take its fastest plan (dtype
    i8 sizes ``w8a16_conv2d``)."""
    nhwc = layout.lower() == "nhwc"
    b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw = conv2d_dims(
        x_shape, w_shape, stride, padding, groups, "nhwc" if nhwc else "nchw")
    prm = _lib.Conv2dParams(kh, kw, sh, sw, ph, pw, groups, 0)
    out = ctypes.c_size_t(0)
    check(lib.teeny_conv2d_workspace_size(b, cin, cout, h, wd, oh, ow, ctypes.byref(prm), from_any(dtype).code,
                                          _lib.NHWC if nhwc else _lib.NCHW, ctypes.byref(out)))
    return int(out.value)


def linear_workspace_size(m: int, n: int, k: int, dtype=bf16) -> int:
    """Stream workspace bytes that let ``linear`` (dtype f32/bf16) or
    ``w8a16_linear`` (dtype i8) take its fastest plan at [m,k] x [n,k]^T."""
    out = ctypes.c_size_t(0)
    check(lib.teeny_linear_workspace_size(m, n, k, from_any(dtype).code, ctypes.byref(out)))
    return int(out.value)


def flash_attention(q: Buffer, k: Buffer, v: Buffer, softmax_scale: Optional[float] = None,
                    causal: bool = False, o: Optional[Buffer] = None, lse: Optional[Buffer] = None,
                    stream: Optional[Stream] = None) -> Buffer:
    """q [BH, Nq, D], k/v [BH, Nk, D] -> o [BH, Nq, D]; lse (fp32 [BH, Nq]) optional."""
    bh, nq, nk, d = attention_dims(q.shape, k.shape, v.shape, lse.shape if lse is not None else None)
    _need(k.dtype == q.dtype and v.dtype == q.dtype, "attention: q/k/v dtypes differ")
    _need(lse is None or lse.dtype == f32, "attention: lse is fp32")
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    o = _out(q, o)
    check(lib.teeny_flash_attention2_forward(q.ptr, k.ptr, v.ptr, o.ptr,
                                             lse.ptr if lse is not None else None, nq, nk, scale,
                                             bh, d, int(bool(causal)), q.dtype.code, _h(stream)))
    return o


def attention(q: Buffer, k: Buffer, v: Buffer, q_heads: int, kv_heads: int,
              softmax_scale: Optional[float] = None, causal: bool = False, o: Optional[Buffer] = None,
              lse: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """Multi-head attention with grouped K/V heads: q [B*q_heads, Nq, D], k/v
    [B*kv_heads, Nk, D] -> o [B*q_heads, Nq, D]."""
    _need(len(q.shape) == 3 and len(k.shape) == 3 and tuple(k.shape) == tuple(v.shape),
          "attention: q [B*Hq, Nq, D], k/v [B*Hkv, Nk, D]")
    _need(q_heads > 0 and kv_heads > 0 and q_heads % kv_heads == 0, "attention: q_heads % kv_heads != 0")
    bhq, nq, d = q.shape
    _need(bhq % q_heads == 0, "attention: q's first dim must be B * q_heads")
    batch = bhq // q_heads
    _need(k.shape[0] == batch * kv_heads and k.shape[2] == d, "attention: k/v must be [B*kv_heads, Nk, D]")
    _need(lse is None or (lse.numel == bhq * nq and lse.dtype == f32), "attention: lse fp32 [B*q_heads, Nq]")
    _need(k.dtype == q.dtype and v.dtype == q.dtype, "attention: q/k/v dtypes differ")
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    o = _out(q, o)
    check(lib.teeny_attention_forward(q.ptr, k.ptr, v.ptr, o.ptr, lse.ptr if lse is not None else None,
                                      batch, q_heads, kv_heads, nq, k.shape[1], d, scale, int(bool(causal)),
                                      q.dtype.code, _h(stream)))
    return o


def attention_backward(q: Buffer, k: Buffer, v: Buffer, o: Buffer, do: Buffer, lse: Buffer,
                       q_heads: int = 1, kv_heads: int = 1, softmax_scale: Optional[float] = None,
                       causal: bool = False, dq: Optional[Buffer] = None, dk: Optional[Buffer] = None,
                       dv: Optional[Buffer] = None, stream: Optional[Stream] = None):
    """flash_attn2.rs:173-447: (dq, dk, dv) from the forward's o and lse (fp32
    logsumexp); q/o/do [B*q_heads, Nq, D], k/v [B*kv_heads, Nk, D]."""
    _need(len(q.shape) == 3 and len(k.shape) == 3 and tuple(k.shape) == tuple(v.shape),
          "attention_backward: q [B*Hq, Nq, D], k/v [B*Hkv, Nk, D]")
    _need(q_heads > 0 and kv_heads > 0 and q_heads % kv_heads == 0, "attention_backward: q_heads % kv_heads != 0")
    bhq, nq, d = q.shape
    _need(bhq % q_heads == 0, "attention_backward: q's first dim must be B * q_heads")
    batch = bhq // q_heads
    _need(k.shape[0] == batch * kv_heads and k.shape[2] == d, "attention_backward: k/v must be [B*kv_heads, Nk, D]")
    _need(tuple(o.shape) == tuple(q.shape) and tuple(do.shape) == tuple(q.shape), "attention_backward: o/do like q")
    _need(all(t.dtype == q.dtype for t in (k, v, o, do)), "attention_backward: dtypes differ")
    _need(lse.numel == bhq * nq and lse.dtype == f32, "attention_backward: lse fp32 [B*q_heads, Nq]")
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    dq, dk, dv = _out(q, dq), _out(k, dk), _out(v, dv)
    check(lib.teeny_attention_backward(q.ptr, k.ptr, v.ptr, o.ptr, do.ptr, lse.ptr, dq.ptr, dk.ptr, dv.ptr, batch,
                                       q_heads, kv_heads, nq, k.shape[1], d, scale, int(bool(causal)),
                                       q.dtype.code, _h(stream)))
    return dq, dk, dv


def flash_attention_backward_dq(q, k, v, o, do, lse, softmax_scale=None, causal=False, dq=None, stream=None):
    """flash_attention2_backward_dq (flash_attn2.rs:173-310): [BH, N, D] tensors."""
    bh, nq, nk, d = attention_dims(q.shape, k.shape, v.shape, lse.shape)
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    dq = _out(q, dq)
    check(lib.teeny_flash_attention2_backward_dq(q.ptr, k.ptr, v.ptr, o.ptr, do.ptr, lse.ptr, dq.ptr, nq, nk, scale,
                                                 bh, d, int(bool(causal)), q.dtype.code, _h(stream)))
    return dq


def flash_attention_backward_dkv(q, k, v, o, do, lse, softmax_scale=None, causal=False, dk=None, dv=None,
                                 stream=None):
    """flash_attention2_backward_dkv (flash_attn2.rs:312-447): [BH, N, D] tensors."""
    bh, nq, nk, d = attention_dims(q.shape, k.shape, v.shape, lse.shape)
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else softmax_scale
    dk, dv = _out(k, dk), _out(v, dv)
    check(lib.teeny_flash_attention2_backward_dkv(q.ptr, k.ptr, v.ptr, o.ptr, do.ptr, lse.ptr, dk.ptr, dv.ptr, nq,
                                                  nk, scale, bh, d, int(bool(causal)), q.dtype.code, _h(stream)))
    return dk, dv


def attention_backward_workspace_size(batch: int, q_heads: int, n_ctx_q: int) -> int:
    out = ctypes.c_size_t(0)
    check(lib.teeny_attention_backward_workspace_size(batch, q_heads, n_ctx_q, ctypes.byref(out)))
    return int(out.value)


GRANULARITY = {"tensor": _lib.PER_TENSOR, "channel": _lib.PER_CHANNEL, "group": _lib.GROUP}


def quant_num_groups(shape, granularity="channel", axis=0, group_size=1) -> int:
    sh = (ctypes.c_int64 * max(1, len(shape)))(*shape)
    out = ctypes.c_int64()
    check(lib.teeny_quant_num_groups(sh, len(shape), GRANULARITY[granularity], axis, group_size,
                                     ctypes.byref(out)))
    return out.value


def quantize_affine(data: Buffer, shape, granularity="channel", axis=0, group_size=1,
                    symmetric=True, bits=8, want_groups=False, stream: Optional[Stream] = None):
    """teeny-quant quantize_affine on the GPU (affine.rs:55-148).  Returns
    (qvalues int8, scales f32, zero_points i32, groups u32 or None)."""
    ng = quant_num_groups(shape, granularity, axis, group_size)
    n = _prod(shape)
    _need(data.dtype == f32 and data.numel == n, f"quantize_affine: data must be fp32 with {n} elements")
    q = Buffer(i8, tuple(shape))
    scales = Buffer(f32, (max(ng, 1),))
    zps = Buffer("i32", (max(ng, 1),))
    groups = Buffer("u32", (n,)) if want_groups else None
    sh = (ctypes.c_int64 * max(1, len(shape)))(*shape)
    check(lib.teeny_quantize_affine(data.ptr, sh, len(shape), GRANULARITY[granularity], axis,
                                    group_size, int(bool(symmetric)), bits, q.ptr, scales.ptr,
                                    zps.ptr, groups.ptr if groups is not None else None, _h(stream)))
    return q, scales, zps, groups


def dequantize_affine(q: Buffer, scales: Buffer, zero_points: Optional[Buffer], shape,
                      granularity="channel", axis=0, group_size=1, out: Optional[Buffer] = None,
                      stream: Optional[Stream] = None) -> Buffer:
    ng = quant_num_groups(shape, granularity, axis, group_size)
    _need(q.numel == _prod(shape) and q.dtype == i8, "dequantize_affine: q must be int8 of the shape")
    _need(scales.numel >= ng and (zero_points is None or zero_points.numel >= ng),
          f"dequantize_affine: scales/zero_points need {ng} entries")
    out = _out(q, out, tuple(shape), f32)
    sh = (ctypes.c_int64 * max(1, len(shape)))(*shape)
    check(lib.teeny_dequantize_affine(q.ptr, scales.ptr,
                                      zero_points.ptr if zero_points is not None else None, sh,
                                      len(shape), GRANULARITY[granularity], axis, group_size,
                                      out.ptr, _h(stream)))
    return out


def linear(x: Buffer, w: Buffer, b: Optional[Buffer] = None, y: Optional[Buffer] = None,
           stream: Optional[Stream] = None) -> Buffer:
    m, n, k = linear_dims(x.shape, w.shape, b.shape if b is not None else None)
    _need(w.dtype == x.dtype and (b is None or b.dtype == x.dtype), "linear: w/b dtype must match x")
    y = _out(x, y, (m, n))
    check(lib.teeny_linear_forward(x.ptr, w.ptr, b.ptr if b is not None else None, y.ptr, m, n, k,
                                   k, 1, k, 1, n, 1, x.dtype.code, _h(stream)))
    return y


def linear_backward(x: Buffer, w: Buffer, dy: Buffer, use_bias: bool = True, dx: Optional[Buffer] = None,
                    dw: Optional[Buffer] = None, db: Optional[Buffer] = None,
                    stream: Optional[Stream] = None) -> Tuple[Buffer, Buffer, Optional[Buffer]]:
    """Gradients of ``linear`` (linear.rs:118-250): x [M,K], w [N,K], dy [M,N]
    -> (dx [M,K] = dy w, dw [N,K] = dy^T x, db [N] = column sums of dy, or
    None without bias).  Written, not accumulated."""
    m, n, k = linear_dims(x.shape, w.shape)
    _need(tuple(dy.shape) == (m, n), f"linear_backward: dy must be [{m}, {n}], is {list(dy.shape)}")
    _need(w.dtype == x.dtype and dy.dtype == x.dtype, "linear_backward: x/w/dy dtypes differ")
    dx = _out(x, dx, (m, k))
    dw = _out(x, dw, (n, k))
    db = _out(x, db, (n,)) if use_bias else None
    check(lib.teeny_linear_backward(x.ptr, w.ptr, dy.ptr, dx.ptr, dw.ptr, db.ptr if db is not None else None,
                                    m, n, k, k, 1, 1, k, n, 1, k, 1, 1, k, 1, x.dtype.code, _h(stream)))
    return dx, dw, db


def linear_backward_workspace_size(m: int, n: int, k: int, dtype=bf16) -> int:
    """Stream workspace bytes that let ``linear_backward`` take its fastest plan."""
    out = ctypes.c_size_t(0)
    check(lib.teeny_linear_backward_workspace_size(m, n, k, from_any(dtype).code, ctypes.byref(out)))
    return int(out.value)


def w8a16_linear(x: Buffer, qweight: Buffer, scale: Buffer, bias: Optional[Buffer] = None,
                 act: Optional[str] = None, y: Optional[Buffer] = None,
                 stream: Optional[Stream] = None) -> Buffer:
    m, n, k = w8a16_dims(x.shape, qweight.shape, scale.shape, bias.shape if bias is not None else None)
    _need(x.dtype == bf16 and qweight.dtype == i8 and scale.dtype == f32 and
          (bias is None or bias.dtype == f32), "w8a16_linear: x bf16, qweight int8, scale/bias fp32")
    y = _out(x, y, (m, n), bf16)
    check(lib.teeny_w8a16_linear_forward(x.ptr, qweight.ptr, scale.ptr,
                                         bias.ptr if bias is not None else None, y.ptr, m, n, k,
                                         ACTS[act], _h(stream)))
    return y


def w8a16_conv2d(x: Buffer, qweight: Buffer, scale: Buffer, bias: Optional[Buffer] = None,
                 stride=(1, 1), padding=(0, 0), groups: int = 1, act: Optional[str] = None,
                 y: Optional[Buffer] = None, stream: Optional[Stream] = None) -> Buffer:
    """x NHWC bf16 [B,H,W,Cin], qweight int8 [Cout,KH,KW,Cin/G], scale f32 [Cout]."""
    b, cin, cout, h, wd, oh, ow, kh, kw, sh, sw, ph, pw = conv2d_dims(
        x.shape, qweight.shape, stride, padding, groups, "nhwc", bias.shape if bias is not None else None)
    _need(_prod(scale.shape) == cout, f"w8a16_conv2d: scale must have {cout} elements")
    _need(x.dtype == bf16 and qweight.dtype == i8 and scale.dtype == f32 and
          (bias is None or bias.dtype == f32), "w8a16_conv2d: x bf16, qweight int8, scale/bias fp32")
    y = _out(x, y, (b, oh, ow, cout), bf16)
    prm = _lib.Conv2dParams(kh, kw, sh, sw, ph, pw, groups, ACTS[act])
    check(lib.teeny_w8a16_conv2d_forward(x.ptr, qweight.ptr, scale.ptr,
                                         bias.ptr if bias is not None else None, y.ptr, b, cin,
                                         cout, h, wd, oh, ow, ctypes.byref(prm), _h(stream)))
    return y
