"""CPU oracle for the teeny-kernels hot path — TEST INFRASTRUCTURE ONLY.

ctypes wrappers over oracle/_build/libteeny_oracle.so, the plain-C
restatement of the reference kernels (oracle/teeny_oracle.c, each function
citing the reference file:line it follows).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or the timed CPU baseline; the product
(teenygrad_amd) never calls it.

Arrays are numpy fp32 (int8/int32/uint32 for quantization).  For bf16
workloads callers pass the bf16-rounded inputs as fp32: the oracle computes
in fp32 on the same values the GPU reads.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libteeny_oracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load(path: str = LIB_PATH) -> ctypes.CDLL:
    if path == LIB_PATH and not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(path)
    P = c_void_p
    I = c_int64
    sigs = {
        "oracle_set_threads": [c_int],
        "oracle_threads": [],
        "oracle_relu_forward": [P, P, I, I, I, I],
        "oracle_gelu_forward": [P, P, I, I, I, I],
        "oracle_silu_forward": [P, P, I, I, I, I],
        "oracle_relu_backward": [P, P, P, I, I, I, I],
        "oracle_gelu_backward": [P, P, P, I, I, I, I],
        "oracle_silu_backward": [P, P, P, I, I, I, I],
        "oracle_sigmoid_forward": [P, P, I, I, I, I],
        "oracle_tanh_forward": [P, P, I, I, I, I],
        "oracle_sigmoid_backward": [P, P, P, I, I, I, I],
        "oracle_tanh_backward": [P, P, P, I, I, I, I],
        "oracle_layer_norm_forward_inference": [P, P, P, P, I, I, c_float, I, I, I],
        "oracle_rms_norm_forward": [P, P, P, P, I, I, c_float, I, I, I],
        "oracle_conv2d_forward": [P, P, P, P] + [I] * 15 + [I, I],
        "oracle_conv2d_bn_silu_forward": [P, P, P, P, P] + [I] * 15 + [I, I],
        "oracle_conv2d_programs": [P, P, P, P] + [I] * 15 + [P, I],
        "oracle_flash_attention2_forward": [P, P, P, P, P, I, I, I, I, c_float, c_int, I, I],
        "oracle_flash_attention2_rows": [P, P, P, P, P, I, I, I, I, c_float, c_int, P, I],
        "oracle_linear_forward": [P, P, P, P] + [I] * 9 + [I, I],
        "oracle_linear_backward": [P] * 6 + [I] * 14,
        "oracle_layer_norm_forward": [P, P, P, P, P, P, I, I, c_float, I, I, I],
        "oracle_layer_norm_backward": [P, P, P, P, P, P, P, P, I, I, I],
        "oracle_rms_norm_backward": [P, P, P, P, P, P, I, I, I],
        "oracle_conv2d_backward_dx": [P, P, P] + [I] * 14,
        "oracle_conv2d_backward_dw": [P, P, P] + [I] * 15,
        "oracle_flash_attention2_backward": [P] * 9 + [I, I, I, I, c_float, c_int],
        "oracle_quant_num_groups": [P, c_int, c_int, c_int, I, POINTER(c_int64)],
        "oracle_quantize_affine": [P, I, P, c_int, c_int, c_int, I, c_int, c_int, P, P, P, P],
        "oracle_dequantize_affine": [P, P, P, P, c_int, c_int, c_int, I, P],
    }
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = c_int
    return lib


lib = _load()
BUILD_FLAGS = "-O3 -march=x86-64-v3 -ffp-contract=off (prebuilt)"


def use_native_build() -> str:
    """Recompiles the oracle for this host (-O3 -march=native, otherwise the
    same flags as oracle/Makefile) in a temporary directory and routes every
    function of this module to it; returns the flags in use.  For timing the
    CPU baseline on the host that runs it; if the compiler is missing or fails,
    the prebuilt library stays in use."""
    global lib, BUILD_FLAGS
    import tempfile
    out = os.path.join(tempfile.mkdtemp(prefix="teeny_oracle_"), "libteeny_oracle_native.so")
    cmd = ["gcc", "-O3", "-std=c11", "-fPIC", "-march=native", "-ffp-contract=off", "-pthread", "-shared",
           os.path.join(HERE, "teeny_oracle.c"), "-o", out, "-lm"]
    try:
        subprocess.run(cmd, check=True, capture_output=True, timeout=120)
        lib = _load(out)
        BUILD_FLAGS = "-O3 -march=native -ffp-contract=off"
    except (OSError, subprocess.SubprocessError):
        pass
    return BUILD_FLAGS


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"oracle {what} failed with status {status}")
        self.status = status


def _chk(rc: int, what: str) -> None:
    if rc != 0:
        raise OracleError(rc, what)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data


def set_threads(n: int) -> None:
    lib.oracle_set_threads(int(n))


def threads() -> int:
    return lib.oracle_threads()


# ── activations (relu.rs:27-64, gelu.rs:31-78, sigmoid.rs:119-158) ────────


def _act(fn, x, block_size, pid_begin, pid_end):
    x = _f32(x)
    y = np.zeros_like(x)
    _chk(fn(_p(x), _p(y), x.size, block_size, pid_begin, pid_end), fn.__name__)
    return y


def relu(x, block_size=1024, pid_begin=0, pid_end=-1):
    return _act(lib.oracle_relu_forward, x, block_size, pid_begin, pid_end)


def gelu(x, block_size=1024, pid_begin=0, pid_end=-1):
    return _act(lib.oracle_gelu_forward, x, block_size, pid_begin, pid_end)


def silu(x, block_size=1024, pid_begin=0, pid_end=-1):
    return _act(lib.oracle_silu_forward, x, block_size, pid_begin, pid_end)


def sigmoid(x, block_size=1024, pid_begin=0, pid_end=-1):
    """sigmoid.rs (sigmoid_forward): 1 / (1 + exp(-x))."""
    return _act(lib.oracle_sigmoid_forward, x, block_size, pid_begin, pid_end)


def tanh(x, block_size=1024, pid_begin=0, pid_end=-1):
    """tanh.rs (tanh_forward): 2 * (1 / (1 + exp(-2x))) - 1."""
    return _act(lib.oracle_tanh_forward, x, block_size, pid_begin, pid_end)


def _act_grad(fn, dy, v, block_size, pid_begin, pid_end):
    dy, v = _f32(dy), _f32(v)
    if dy.shape != v.shape:
        raise ValueError(f"{fn.__name__}: dy {dy.shape} and saved tensor {v.shape} differ")
    dx = np.zeros_like(dy)
    _chk(fn(_p(dy), _p(v), _p(dx), dy.size, block_size, pid_begin, pid_end), fn.__name__)
    return dx


def relu_backward(dy, y, block_size=1024, pid_begin=0, pid_end=-1):
    """relu.rs:67-117: dx = dy where the forward OUTPUT y > 0, else 0."""
    return _act_grad(lib.oracle_relu_backward, dy, y, block_size, pid_begin, pid_end)


def gelu_backward(dy, x, block_size=1024, pid_begin=0, pid_end=-1):
    """gelu.rs:81-139: tanh-GELU derivative at the forward input x, times dy."""
    return _act_grad(lib.oracle_gelu_backward, dy, x, block_size, pid_begin, pid_end)


def silu_backward(dy, x, block_size=1024, pid_begin=0, pid_end=-1):
    """sigmoid.rs:161-210: dy * (s + y - y s), s = sigmoid(x), y = x s."""
    return _act_grad(lib.oracle_silu_backward, dy, x, block_size, pid_begin, pid_end)


def sigmoid_backward(dy, y, block_size=1024, pid_begin=0, pid_end=-1):
    """sigmoid.rs (sigmoid_backward): dy * (y - y y) at the forward OUTPUT y."""
    return _act_grad(lib.oracle_sigmoid_backward, dy, y, block_size, pid_begin, pid_end)


def tanh_backward(dy, y, block_size=1024, pid_begin=0, pid_end=-1):
    """tanh.rs (tanh_backward): dy * (1 - y y) at the forward OUTPUT y."""
    return _act_grad(lib.oracle_tanh_backward, dy, y, block_size, pid_begin, pid_end)


MEMBERS = {"relu": relu, "gelu": gelu, "silu": silu, "sigmoid": sigmoid, "tanh": tanh}
Y_STYLE_GRADS = {"relu": relu_backward, "sigmoid": sigmoid_backward, "tanh": tanh_backward}


def pointwise_chain(x, members, round_fn=None):
    """PointwiseFuse (graph/optimizer/ops/pointwise_fuse.rs:73-233, the
    synthesized entry in -> m0 -> scratch0 -> ... -> out): the members' own
    kernels run in order, each reading the previous member's stored output;
    round_fn (e.g. a bf16 rounding) models a narrower scratch dtype.
    Returns (y, [scratch_0 .. scratch_{n-2}])."""
    outs = []
    v = _f32(x)
    for name in members:
        v = MEMBERS[name](v)
        if round_fn is not None:
            v = round_fn(v)
        outs.append(v)
    return outs[-1], outs[:-1]


def pointwise_chain_backward(dy, y, scratch, members, round_fn=None):
    """The fused backward entry (pointwise_fuse.rs:352-380): dx = dy, then the
    members' y-style gradients from the last to the first, member i reading
    its forward output (y for the last, scratch_i otherwise)."""
    g = _f32(dy)
    outs = list(scratch) + [y]
    for i in range(len(members) - 1, -1, -1):
        g = Y_STYLE_GRADS[members[i]](g, outs[i])
        if round_fn is not None:
            g = round_fn(g)
    return g


# ── norms (layernorm.rs:42-157, rmsnorm.rs:39-119) ──────────────────────────


def layer_norm(x, weight, bias, eps=1e-5, block_n=1024, pid_begin=0, pid_end=-1):
    x = _f32(x)
    w, b = _f32(weight), _f32(bias)
    n = x.shape[-1]
    m = x.size // n
    y = np.zeros_like(x)
    _chk(lib.oracle_layer_norm_forward_inference(_p(x), _p(y), _p(w), _p(b), m, n, eps, block_n,
                                                 pid_begin, pid_end), "layer_norm")
    return y


def rms_norm(x, weight, eps=1e-8, block_n=1024, pid_begin=0, pid_end=-1):
    x = _f32(x)
    w = _f32(weight)
    n = x.shape[-1]
    m = x.size // n
    y = np.zeros_like(x)
    rrms = np.zeros(m, dtype=np.float32)
    _chk(lib.oracle_rms_norm_forward(_p(x), _p(y), _p(w), _p(rrms), m, n, eps, block_n, pid_begin,
                                     pid_end), "rms_norm")
    return y, rrms


# ── conv2d (conv2d.rs:43-156, :642-764) ─────────────────────────────────────


def conv2d_nchw(x, w, bias=None, stride=(1, 1), padding=(0, 0), groups=1, block_ow=16,
                pid_begin=0, pid_end=-1):
    """x [B,Cin,H,W], w [Cout,Cin/G,KH,KW] -> y [B,Cout,OH,OW] (fp32)."""
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    sh, sw = (stride, stride) if isinstance(stride, int) else stride
    ph, pw = (padding, padding) if isinstance(padding, int) else padding
    B, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    y = np.zeros((B, Cout, OH, OW), dtype=np.float32)
    _chk(lib.oracle_conv2d_forward(_p(x), _p(w), _p(bias), _p(y), B, Cin, Cout, H, W, OH, OW, KH, KW,
                                   sh, sw, ph, pw, groups, block_ow, pid_begin, pid_end), "conv2d")
    return y


def conv2d_bn_silu_nchw(x, w, bn_scale, bn_shift, stride=(1, 1), padding=(0, 0), groups=1, block_ow=16,
                        pid_begin=0, pid_end=-1):
    """conv2d_bn_silu.rs:40-199: silu(bn_scale[c] * conv(x, w) + bn_shift[c]), NCHW fp32."""
    x, w = _f32(x), _f32(w)
    sc, sh_ = _f32(bn_scale), _f32(bn_shift)
    sh, sw = (stride, stride) if isinstance(stride, int) else stride
    ph, pw = (padding, padding) if isinstance(padding, int) else padding
    B, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    y = np.zeros((B, Cout, OH, OW), np.float32)
    _chk(lib.oracle_conv2d_bn_silu_forward(_p(x), _p(w), _p(sc), _p(sh_), _p(y), B, Cin, Cout, H, W, OH, OW, KH, KW,
                                           sh, sw, ph, pw, groups, block_ow, pid_begin, pid_end), "conv2d_bn_silu")
    return y


def conv2d_nhwc(x, w, bias=None, stride=(1, 1), padding=(0, 0), groups=1):
    """x [B,H,W,Cin], w [Cout,KH,KW,Cin/G] -> y [B,OH,OW,Cout], via the NCHW restatement."""
    y = conv2d_nchw(np.transpose(x, (0, 3, 1, 2)), np.transpose(w, (0, 3, 1, 2)), bias, stride,
                    padding, groups)
    return np.ascontiguousarray(np.transpose(y, (0, 2, 3, 1)))


def conv2d_nhwc_pixels(x, w, pixels, bias=None, stride=(1, 1), padding=(0, 0), groups=1):
    """Output pixels ``pixels`` (flat indices m = (b*OH + oh)*OW + ow of the
    NHWC output) of conv2d_nhwc, all channels: -> [len(pixels), Cout].  Runs
    only the reference programs (b, c_out, oh, ow) those pixels need, with
    BLOCK_OW = 1 (a tiling constant of the reference that does not change the
    per-pixel arithmetic)."""
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    xn = np.ascontiguousarray(np.transpose(x, (0, 3, 1, 2)))
    wn = np.ascontiguousarray(np.transpose(w, (0, 3, 1, 2)))
    sh, sw = (stride, stride) if isinstance(stride, int) else stride
    ph, pw = (padding, padding) if isinstance(padding, int) else padding
    B, Cin, H, W = xn.shape
    Cout, _, KH, KW = wn.shape
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    pixels = np.asarray(pixels, dtype=np.int64).reshape(-1)
    if pixels.size and (pixels.min() < 0 or pixels.max() >= B * OH * OW):
        raise ValueError("conv2d_nhwc_pixels: pixel index out of range")
    b, rest = np.divmod(pixels, OH * OW)
    oh, ow = np.divmod(rest, OW)
    co = np.arange(Cout, dtype=np.int64)
    # program id ((b * Cout + co) * OH + oh) * OW + ow with BLOCK_OW = 1
    pids = np.ascontiguousarray((((b[:, None] * Cout + co[None, :]) * OH + oh[:, None]) * OW
                                 + ow[:, None]).reshape(-1))
    y = np.zeros((B, Cout, OH, OW), dtype=np.float32)
    _chk(lib.oracle_conv2d_programs(_p(xn), _p(wn), _p(bias), _p(y), B, Cin, Cout, H, W, OH, OW,
                                    KH, KW, sh, sw, ph, pw, groups, 1, _p(pids), pids.size),
         "conv2d_programs")
    return np.ascontiguousarray(y[b[:, None], co[None, :], oh[:, None], ow[:, None]])


# ── attention (flash_attn2.rs:52-158) ───────────────────────────────────────


def flash_attention(q, k, v, softmax_scale=None, causal=False, pid_begin=0, pid_end=-1):
    """q [BH,Nq,D], k/v [BH,Nk,D] -> (o [BH,Nq,D], l [BH,Nq])."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, nq, D = q.shape
    nk = k.shape[1]
    scale = 1.0 / np.sqrt(D) if softmax_scale is None else softmax_scale
    o = np.zeros_like(q)
    l = np.zeros((BH, nq), dtype=np.float32)
    _chk(lib.oracle_flash_attention2_forward(_p(q), _p(k), _p(v), _p(o), _p(l), BH, nq, nk, D,
                                             scale, int(causal), pid_begin, pid_end), "flash_attention")
    return o, l


def flash_attention_rows(q, k, v, rows, softmax_scale=None, causal=False):
    """Only program ids `rows` (= bh * Nq + q_row); returns (o_rows [n,D], l_rows [n])."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, nq, D = q.shape
    nk = k.shape[1]
    scale = 1.0 / np.sqrt(D) if softmax_scale is None else softmax_scale
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    o = np.zeros_like(q)
    l = np.zeros((BH, nq), dtype=np.float32)
    _chk(lib.oracle_flash_attention2_rows(_p(q), _p(k), _p(v), _p(o), _p(l), BH, nq, nk, D, scale,
                                          int(causal), _p(rows), rows.size), "flash_attention_rows")
    return o.reshape(-1, D)[rows], l.reshape(-1)[rows]


# ── linear (linear.rs:20-116) ───────────────────────────────────────────────


def linear(x, w, b=None, pid_begin=0, pid_end=-1):
    x, w = _f32(x), _f32(w)
    b = None if b is None else _f32(b)
    M, K = x.shape
    N = w.shape[0]
    y = np.zeros((M, N), dtype=np.float32)
    _chk(lib.oracle_linear_forward(_p(x), _p(w), _p(b), _p(y), M, N, K, K, 1, K, 1, N, 1, pid_begin,
                                   pid_end), "linear")
    return y


def linear_backward(x, w, dy, use_bias=True):
    """linear.rs:118-250: x [M,K], w [N,K], dy [M,N] -> (dx [M,K], dw [N,K],
    db [N] or None), contiguous operands."""
    x, w, dy = _f32(x), _f32(w), _f32(dy)
    M, K = x.shape
    N = w.shape[0]
    dx = np.zeros((M, K), np.float32)
    dw = np.zeros((N, K), np.float32)
    db = np.zeros(N, np.float32) if use_bias else None
    _chk(lib.oracle_linear_backward(_p(x), _p(w), _p(dy), _p(dx), _p(dw), _p(db), M, N, K, K, 1, 1, K, N, 1,
                                    K, 1, 1, K, 1), "linear_backward")
    return dx, dw, db


# ── training: saved statistics and backward kernels ─────────────────────────


def layer_norm_train(x, weight, bias, eps=1e-5, block_n=1024):
    """layernorm.rs:162-298: (y, mean [M], rstd [M])."""
    x = _f32(x)
    w, b = _f32(weight), _f32(bias)
    n = x.shape[-1]
    m = x.size // n
    y = np.zeros_like(x)
    mean = np.zeros(m, np.float32)
    rstd = np.zeros(m, np.float32)
    _chk(lib.oracle_layer_norm_forward(_p(x), _p(y), _p(w), _p(b), _p(mean), _p(rstd), m, n, eps, block_n, 0, -1),
         "layer_norm_train")
    return y, mean, rstd


def layer_norm_backward(dy, x, weight, mean, rstd, dweight=None, dbias=None, block_n=1024):
    """layernorm.rs:300-482: (dx, dweight, dbias); dweight/dbias accumulate
    into the given arrays (zeros when None), rows in order."""
    dy, x, w = _f32(dy), _f32(x), _f32(weight)
    n = x.shape[-1]
    m = x.size // n
    dx = np.zeros_like(x)
    dw = np.zeros(n, np.float32) if dweight is None else _f32(dweight).copy()
    db = np.zeros(n, np.float32) if dbias is None else _f32(dbias).copy()
    _chk(lib.oracle_layer_norm_backward(_p(dy), _p(x), _p(dx), _p(w), _p(dw), _p(db), _p(_f32(mean)),
                                        _p(_f32(rstd)), m, n, block_n), "layer_norm_backward")
    return dx, dw, db


def rms_norm_backward(dy, x, weight, rrms, dweight=None, block_n=1024):
    """rmsnorm.rs:135-277: (dx, dweight), dweight accumulated as above."""
    dy, x, w = _f32(dy), _f32(x), _f32(weight)
    n = x.shape[-1]
    m = x.size // n
    dx = np.zeros_like(x)
    dw = np.zeros(n, np.float32) if dweight is None else _f32(dweight).copy()
    _chk(lib.oracle_rms_norm_backward(_p(dy), _p(x), _p(dx), _p(w), _p(dw), _p(_f32(rrms)), m, n, block_n),
         "rms_norm_backward")
    return dx, dw


def _conv_geo(x_shape, w_shape, stride, padding):
    sh, sw = (stride, stride) if isinstance(stride, int) else stride
    ph, pw = (padding, padding) if isinstance(padding, int) else padding
    B, Cin, H, W = x_shape
    Cout, _, KH, KW = w_shape
    return B, Cin, Cout, H, W, (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1, KH, KW, sh, sw, ph, pw


def conv2d_backward_dx(dy, w, x_shape, stride=(1, 1), padding=(0, 0), groups=1):
    """conv2d.rs:171-284, NCHW: dx [B, Cin, H, W]."""
    dy, w = _f32(dy), _f32(w)
    B, Cin, Cout, H, W, OH, OW, KH, KW, sh, sw, ph, pw = _conv_geo(x_shape, w.shape, stride, padding)
    dx = np.zeros(tuple(x_shape), np.float32)
    _chk(lib.oracle_conv2d_backward_dx(_p(dy), _p(w), _p(dx), B, Cin, Cout, H, W, OH, OW, KH, KW, sh, sw, ph, pw,
                                       groups), "conv2d_backward_dx")
    return dx


def conv2d_backward_dw(dy, x, w_shape, stride=(1, 1), padding=(0, 0), groups=1, block_ow=16):
    """conv2d.rs:286-397, NCHW: dw [Cout, Cin/G, KH, KW]."""
    dy, x = _f32(dy), _f32(x)
    B, Cin, Cout, H, W, OH, OW, KH, KW, sh, sw, ph, pw = _conv_geo(x.shape, w_shape, stride, padding)
    dw = np.zeros(tuple(w_shape), np.float32)
    _chk(lib.oracle_conv2d_backward_dw(_p(dy), _p(x), _p(dw), B, Cin, Cout, H, W, OH, OW, KH, KW, sh, sw, ph, pw,
                                       groups, block_ow), "conv2d_backward_dw")
    return dw


def flash_attention_backward(q, k, v, o, do, l, softmax_scale=None, causal=False):
    """flash_attn2.rs:173-447: (dq, dk, dv) for [BH, N, D] tensors, L the
    forward's logsumexp [BH, Nq]."""
    q, k, v, o, do, l = (_f32(a) for a in (q, k, v, o, do, l))
    BH, nq, D = q.shape
    nk = k.shape[1]
    scale = 1.0 / np.sqrt(D) if softmax_scale is None else softmax_scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    _chk(lib.oracle_flash_attention2_backward(_p(q), _p(k), _p(v), _p(o), _p(do), _p(l), _p(dq), _p(dk), _p(dv),
                                              BH, nq, nk, D, scale, int(causal)), "flash_attention_backward")
    return dq, dk, dv


# ── teeny-quant (affine.rs:47-161, groups.rs:20-100) ───────────────────────

GRAN = {"tensor": 0, "channel": 1, "group": 2}


def quant_num_groups(shape, granularity="channel", axis=0, group_size=1) -> int:
    sh = np.ascontiguousarray(shape, dtype=np.int64)
    out = c_int64()
    _chk(lib.oracle_quant_num_groups(_p(sh), len(shape), GRAN[granularity], axis, group_size,
                                     ctypes.byref(out)), "quant_num_groups")
    return out.value


def quantize_affine(data, shape, granularity="channel", axis=0, group_size=1, symmetric=True,
                    bits=8):
    """Returns (qvalues int8, scales f32, zero_points i32, groups u32)."""
    data = _f32(data).reshape(-1)
    sh = np.ascontiguousarray(shape, dtype=np.int64)
    ng = quant_num_groups(shape, granularity, axis, group_size)
    n = int(np.prod(shape)) if len(shape) else 1
    q = np.zeros(max(n, data.size), dtype=np.int8)
    scales = np.zeros(max(ng, 1), dtype=np.float32)
    zps = np.zeros(max(ng, 1), dtype=np.int32)
    groups = np.zeros(max(n, 1), dtype=np.uint32)
    _chk(lib.oracle_quantize_affine(_p(data), data.size, _p(sh), len(shape), GRAN[granularity],
                                    axis, group_size, int(bool(symmetric)), bits, _p(q),
                                    _p(scales), _p(zps), _p(groups)), "quantize_affine")
    return q[:n], scales[:ng], zps[:ng], groups[:n]


def dequantize_affine(q, scales, zero_points, shape, granularity="channel", axis=0, group_size=1):
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales = _f32(scales)
    zps = None if zero_points is None else np.ascontiguousarray(zero_points, dtype=np.int32)
    sh = np.ascontiguousarray(shape, dtype=np.int64)
    out = np.zeros(int(np.prod(shape)) if len(shape) else 1, dtype=np.float32)
    _chk(lib.oracle_dequantize_affine(_p(q), _p(scales), _p(zps), _p(sh), len(shape),
                                      GRAN[granularity], axis, group_size, _p(out)),
         "dequantize_affine")
    return out.reshape(shape)


def w8a16_linear(x, q, scales, bias=None):
    """linear_forward on dequantize_affine's weights (per-channel axis 0)."""
    w = dequantize_affine(q, scales, None, q.shape, "channel", 0)
    return linear(x, w, bias)
