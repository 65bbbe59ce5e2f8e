"""The C ABI without a GPU: exports, and the error paths of every entry point.

Every argument check of include/teeny_hip.h happens on the host before any
HIP call, so these run in a container without a device.  Pointers passed
here are never dereferenced (the calls are rejected first).
"""
import ctypes
import os
import re

import pytest

import teenygrad_amd as tg
from teenygrad_amd import _lib
from teenygrad_amd._lib import lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "teeny_hip.h")
FAKE = 0x100000  # 16-byte aligned, never dereferenced
FAKE_ODD = 0x100002


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:teeny_status|const char \*)\s*(teeny_\w+)\(", text, re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    names = header_functions()
    assert len(names) >= 40
    so = ctypes.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(so, n), f"{n} declared in teeny_hip.h but not exported"
        assert n in _lib.EXPORTED, f"{n} not bound in teenygrad_amd/_lib.py"
    assert set(_lib.EXPORTED) == set(names)


def test_status_strings_and_version():
    assert lib.teeny_status_string(0) == b"ok"
    assert lib.teeny_status_string(_lib.ERR_NULL_POINTER) == b"null pointer"
    assert b"gfx950" in lib.teeny_hip_version()


def expect(status, code):
    assert status == code, f"status {status} ({tg._lib.last_error()}), wanted {code}"
    assert tg._lib.last_error() != ""


@pytest.mark.parametrize("fn", ["teeny_relu_forward", "teeny_gelu_forward", "teeny_silu_forward"])
def test_activation_errors(fn):
    f = getattr(lib, fn)
    expect(f(None, FAKE, 10, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(f(FAKE, FAKE, -1, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(f(FAKE, FAKE, 10, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    expect(f(FAKE, FAKE, 10, 99, None), _lib.ERR_UNSUPPORTED_DTYPE)
    assert f(None, None, 0, _lib.F32, None) == _lib.OK  # empty tensor is a no-op


@pytest.mark.parametrize("fn", ["teeny_relu_backward", "teeny_gelu_backward", "teeny_silu_backward"])
def test_activation_backward_errors(fn):
    f = getattr(lib, fn)
    expect(f(None, FAKE, FAKE, 10, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(f(FAKE, None, FAKE, 10, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(f(FAKE, FAKE, None, 10, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    expect(f(FAKE, FAKE, FAKE, -1, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(f(FAKE, FAKE, FAKE, 10, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    assert f(None, None, None, 0, _lib.F32, None) == _lib.OK  # empty tensor is a no-op


def test_norm_errors():
    ln = lib.teeny_layer_norm_forward_inference
    expect(ln(FAKE, FAKE, FAKE, None, 4, 8, 1e-5, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(ln(FAKE, FAKE, FAKE, FAKE, 4, 0, 1e-5, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(ln(FAKE, FAKE, FAKE, FAKE, -4, 8, 1e-5, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(ln(FAKE, FAKE, FAKE, FAKE, 4, 8, 1e-5, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    rms = lib.teeny_rms_norm_forward
    expect(rms(FAKE, FAKE, None, None, 4, 8, 1e-8, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    na = lib.teeny_norm_act_forward
    expect(na(FAKE, FAKE, FAKE, FAKE, 4, 8, 1e-5, 0, 17, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    assert ln(None, None, None, None, 0, 8, 1e-5, _lib.F32, None) == _lib.OK


def conv_params(kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, g=1, act=0):
    return ctypes.byref(_lib.Conv2dParams(kh, kw, sh, sw, ph, pw, g, act))


def test_conv_errors():
    c = lib.teeny_conv2d_forward
    # OH/OW inconsistent with (H + 2p - k)/s + 1
    expect(c(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 7, 8, conv_params(), _lib.F32, _lib.NCHW, None),
           _lib.ERR_SHAPE_MISMATCH)
    # groups must divide channels
    expect(c(FAKE, FAKE, FAKE, 1, 4, 6, 8, 8, 8, 8, conv_params(g=4), _lib.F32, _lib.NCHW, None),
           _lib.ERR_SHAPE_MISMATCH)
    expect(c(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(sh=0), _lib.F32, _lib.NCHW, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(c(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, None, _lib.F32, _lib.NCHW, None),
           _lib.ERR_NULL_POINTER)
    expect(c(None, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, _lib.NCHW, None),
           _lib.ERR_NULL_POINTER)
    expect(c(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.I8, _lib.NCHW, None),
           _lib.ERR_UNSUPPORTED_DTYPE)
    expect(c(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, 5, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_conv2d_bias_forward(FAKE, FAKE, None, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(),
                                         _lib.F32, _lib.NCHW, None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_w8a16_conv2d_forward(FAKE, FAKE, None, None, FAKE, 1, 16, 16, 8, 8, 8, 8,
                                          conv_params(), None), _lib.ERR_NULL_POINTER)


def test_attention_errors():
    fa = lib.teeny_flash_attention2_forward
    expect(fa(FAKE, FAKE, FAKE, FAKE, None, 8, 0, 0.125, 4, 64, 0, _lib.F32, None),
           _lib.ERR_SHAPE_MISMATCH)
    expect(fa(FAKE, FAKE, FAKE, FAKE, None, 8, 8, 0.125, 4, 96, 0, _lib.BF16, None),
           _lib.ERR_UNSUPPORTED)
    expect(fa(FAKE, FAKE, FAKE, FAKE, None, 8, 8, 0.125, 4, 48, 0, _lib.F32, None),
           _lib.ERR_UNSUPPORTED)
    expect(fa(FAKE_ODD, FAKE, FAKE, FAKE, None, 8, 8, 0.125, 4, 128, 0, _lib.BF16, None),
           _lib.ERR_MISALIGNED)
    expect(fa(FAKE, None, FAKE, FAKE, None, 8, 8, 0.125, 4, 64, 0, _lib.F32, None),
           _lib.ERR_NULL_POINTER)
    expect(fa(FAKE, FAKE, FAKE, FAKE, None, 8, 8, 0.125, 4, 64, 0, _lib.I8, None),
           _lib.ERR_UNSUPPORTED_DTYPE)
    # bf16 K/V of one head are addressed with 32-bit offsets: 2^23 keys of 128 bf16 are 2 GiB
    expect(fa(FAKE, FAKE, FAKE, FAKE, None, 8, 1 << 23, 0.125, 4, 128, 0, _lib.BF16, None),
           _lib.ERR_SHAPE_MISMATCH)


def shape_arr(*s):
    return (ctypes.c_int64 * len(s))(*s)


def test_quant_errors_and_group_count():
    ng = ctypes.c_int64()
    assert lib.teeny_quant_num_groups(shape_arr(8, 5, 33), 3, _lib.GROUP, 2, 8, ctypes.byref(ng)) == 0
    assert ng.value == 8 * 5 * 5
    assert lib.teeny_quant_num_groups(shape_arr(11008, 4096), 2, _lib.PER_CHANNEL, 0, 1,
                                      ctypes.byref(ng)) == 0 and ng.value == 11008
    q = lib.teeny_quantize_affine
    # affine.rs:72-87: axis out of range -> InvalidAxis, group_size 0 -> InvalidGroupSize
    expect(q(FAKE, shape_arr(4), 1, _lib.PER_CHANNEL, 3, 1, 1, 8, FAKE, FAKE, FAKE, None, None),
           _lib.ERR_INVALID_AXIS)
    expect(q(FAKE, shape_arr(4), 1, _lib.GROUP, 0, 0, 1, 8, FAKE, FAKE, FAKE, None, None),
           _lib.ERR_INVALID_GROUP_SIZE)
    expect(q(FAKE, shape_arr(4), 1, _lib.PER_TENSOR, 0, 1, 1, 9, FAKE, FAKE, FAKE, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(q(FAKE, shape_arr(4), 1, _lib.PER_TENSOR, 0, 1, 1, 8, FAKE, None, FAKE, None, None),
           _lib.ERR_NULL_POINTER)
    expect(q(FAKE, shape_arr(4), 1, 7, 0, 1, 1, 8, FAKE, FAKE, FAKE, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_dequantize_affine(FAKE, FAKE, None, shape_arr(4, 4), 2, _lib.PER_CHANNEL, 2, 1,
                                       FAKE, None), _lib.ERR_INVALID_AXIS)


def test_linear_errors():
    li = lib.teeny_linear_forward
    expect(li(FAKE, FAKE, None, None, 4, 4, 4, 4, 1, 4, 1, 4, 1, _lib.F32, None),
           _lib.ERR_NULL_POINTER)
    expect(li(FAKE, FAKE, None, FAKE, 4, 4, 4, 4, 1, 4, 1, 4, 1, _lib.I8, None),
           _lib.ERR_UNSUPPORTED_DTYPE)
    w8 = lib.teeny_w8a16_linear_forward
    expect(w8(FAKE, FAKE, None, None, FAKE, 4, 4, 16, 0, None), _lib.ERR_NULL_POINTER)
    expect(w8(FAKE, FAKE, FAKE, None, FAKE, -1, 4, 16, 0, None), _lib.ERR_SHAPE_MISMATCH)
    expect(w8(FAKE, FAKE, FAKE, None, FAKE, 4, 4, 16, 9, None), _lib.ERR_INVALID_ARGUMENT)
    lb = lib.teeny_linear_backward
    strides = (4, 1, 1, 4, 4, 1, 4, 1, 1, 4, 1)
    expect(lb(FAKE, FAKE, FAKE, None, FAKE, None, 4, 4, 4, *strides, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(lb(FAKE, FAKE, FAKE, FAKE, None, None, 4, 4, 4, *strides, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(lb(FAKE, None, FAKE, FAKE, FAKE, None, 4, 4, 4, *strides, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(lb(FAKE, FAKE, FAKE, FAKE, FAKE, None, -1, 4, 4, *strides, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(lb(FAKE, FAKE, FAKE, FAKE, FAKE, None, 4, 2 ** 31, 4, *strides, _lib.F32, None),
           _lib.ERR_SHAPE_MISMATCH)
    expect(lb(FAKE, FAKE, FAKE, FAKE, FAKE, None, 4, 4, 4, *strides, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    size = ctypes.c_size_t(1)
    assert lib.teeny_linear_backward_workspace_size(64, 48, 64, _lib.F32, ctypes.byref(size)) == _lib.OK
    assert size.value == 0  # fp32 takes the generic kernel: no scratch
    assert lib.teeny_linear_backward_workspace_size(64, 30, 64, _lib.BF16, ctypes.byref(size)) == _lib.OK
    assert size.value == 0  # N % 8 != 0: generic kernel
    expect(lib.teeny_linear_backward_workspace_size(4, 4, 4, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_linear_backward_workspace_size(-4, 4, 4, _lib.BF16, ctypes.byref(size)), _lib.ERR_SHAPE_MISMATCH)


def packed(*kinds_values):
    arr = (_lib.TeenyArg * len(kinds_values))()
    for a, (k, v) in zip(arr, kinds_values):
        a.kind = k
        setattr(a.v, {_lib.ARG_PTR: "ptr", _lib.ARG_I32: "i32", _lib.ARG_F32: "f32"}[k], v)
    return arr


def test_dispatch_errors():
    d = lib.teeny_dispatch
    cg = (ctypes.c_int64 * 1)(1024)
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    args = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_I32, 8))
    expect(d(b"softmax_forward_entry_point", cg, 1, args, 3, grid, _lib.F32, None), _lib.ERR_NOT_FOUND)
    # wrong kind in position 2 (f32 instead of i32)
    bad = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_F32, 8.0))
    expect(d(b"relu_forward_entry_point", cg, 1, bad, 3, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    # missing and trailing arguments
    expect(d(b"relu_forward_entry_point", cg, 1, args, 2, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    extra = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_I32, 8), (_lib.ARG_I32, 1))
    expect(d(b"relu_forward_entry_point", cg, 1, extra, 4, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    # const generics count
    expect(d(b"conv2d_forward_entry_point", cg, 1, args, 3, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    # a rejected op through dispatch keeps the op's own status
    neg = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_I32, -3))
    expect(d(b"relu_forward_entry_point", cg, 1, neg, 3, grid, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)


@pytest.mark.parametrize("op", [b"relu_backward", b"gelu_backward", b"silu_backward"])
def test_dispatch_backward_argument_list(op):
    # (dy_ptr, y_ptr | x_ptr, dx_ptr, n_elements), BLOCK_SIZE: relu.rs:156-172 etc.
    d = lib.teeny_dispatch
    ep = op + b"_entry_point"
    cg = (ctypes.c_int64 * 1)(1024)
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    fwd_shaped = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_I32, 8))
    expect(d(ep, cg, 1, fwd_shaped, 3, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    null_dx = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, None), (_lib.ARG_I32, 8))
    expect(d(ep, cg, 1, null_dx, 4, grid, _lib.F32, None), _lib.ERR_NULL_POINTER)
    neg = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_I32, -1))
    expect(d(ep, cg, 1, neg, 4, grid, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(d(ep, cg, 0, neg, 4, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)  # no BLOCK_SIZE
    empty = packed((_lib.ARG_PTR, None), (_lib.ARG_PTR, None), (_lib.ARG_PTR, None), (_lib.ARG_I32, 0))
    assert d(ep, cg, 1, empty, 4, grid, _lib.BF16, None) == _lib.OK


def test_no_device_paths():
    if tg.device_count() > 0:
        pytest.skip("a device is visible")
    expect(lib.teeny_hip_device_open(0), _lib.ERR_NO_DEVICE)


def test_workspace_registry_and_sizes():
    # attaching is validated on the host; detaching (NULL / 0) always succeeds
    assert lib.teeny_hip_stream_set_workspace(None, FAKE_ODD, 4096) == _lib.ERR_MISALIGNED
    assert lib.teeny_hip_stream_set_workspace(None, None, 0) == 0
    out = ctypes.c_size_t(7)
    assert lib.teeny_linear_workspace_size(4, 4, 4, _lib.BF16, None) == _lib.ERR_NULL_POINTER
    assert lib.teeny_linear_workspace_size(-1, 4, 4, _lib.BF16, ctypes.byref(out)) == _lib.ERR_SHAPE_MISMATCH
    # sizes are pure functions of the shape (a 256-CU device is assumed without a GPU)
    if tg.device_count() == 0:
        # 64 x 256 x 4096 bf16: 2 tiles of 128 x 128, K split 4 ways -> 4 fp32 slices of 64 x 256
        assert tg.kernels.linear_workspace_size(64, 256, 4096, tg.bf16) == 4 * 64 * 256 * 4
        # 64 x 64 x 4096 int8: 1 tile of 128 x 64 -> 4 slices of 64 x 64
        assert tg.kernels.linear_workspace_size(64, 64, 4096, tg.i8) == 4 * 64 * 64 * 4
        # int8 weights are converted in registers on every path (no dequantized
        # copy): the two configuration GEMMs need no scratch at all
        assert tg.kernels.linear_workspace_size(4096, 11008, 4096, tg.i8) == 0
        assert tg.kernels.linear_workspace_size(4096, 4096, 11008, tg.i8) == 0
        assert tg.kernels.linear_workspace_size(4096, 11008, 4096, tg.bf16) == 0
        assert tg.kernels.linear_workspace_size(600, 96, 128, tg.i8) == 0
        # the W8A16 3x3 convs whose shape the band-tiled kernel takes: a bf16
        # copy of the int8 weights (256 x 9 x 256 x 2 B)
        assert tg.kernels.conv2d_workspace_size((32, 28, 28, 256), (256, 3, 3, 256), 1, 1, 1, tg.i8) == 256 * 9 * 256 * 2
        assert tg.kernels.conv2d_workspace_size((128, 28, 28, 256), (256, 3, 3, 256), 1, 1, 1, tg.i8) == 256 * 9 * 256 * 2
        # stride-2 3x3 conv, 3 channels, 20 x 20 -> 10 x 10: space-to-depth input
        # [1, 11, 11, 16] bf16 (3872 B -> 4096) then weights [16, 2, 2, 16] bf16 (2048 B)
        assert tg.kernels.conv2d_workspace_size((1, 20, 20, 3), (16, 3, 3, 3), 2, 1, 1, tg.bf16) == 4096 + 2048
        # fp32 and NCHW convs never use scratch
        assert tg.kernels.conv2d_workspace_size((1, 20, 20, 3), (16, 3, 3, 3), 2, 1, 1, tg.f32) == 0
        assert tg.kernels.conv2d_workspace_size((1, 3, 20, 20), (16, 3, 3, 3), 2, 1, 1, tg.bf16, "nchw") == 0


def test_module_and_launch_errors():
    # validation before any HIP call (drivers/teeny-cuda/src/device/mod.rs:430-490 is the
    # reference's launch; here the checks are the C ABI's own)
    h = ctypes.c_void_p()
    expect(lib.teeny_hip_module_load(None, b"x.hsaco"), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_module_load(ctypes.byref(h), None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_module_load_data(ctypes.byref(h), None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_module_get_function(ctypes.byref(h), None, b"k"), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_module_get_function(ctypes.byref(h), FAKE, None), _lib.ERR_NULL_POINTER)
    assert lib.teeny_hip_module_unload(None) == _lib.OK
    g = (ctypes.c_uint32 * 3)(1, 1, 1)
    b = (ctypes.c_uint32 * 3)(64, 1, 1)
    expect(lib.teeny_hip_launch(None, g, b, 0, None, None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_launch(FAKE, None, b, 0, None, None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_launch(FAKE, (ctypes.c_uint32 * 3)(0, 1, 1), b, 0, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_hip_launch(FAKE, g, (ctypes.c_uint32 * 3)(0, 1, 1), 0, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_hip_launch(FAKE, g, (ctypes.c_uint32 * 3)(1025, 1, 1), 0, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    # 65536 * 65536 wraps to 0 in 32 bits: must still be rejected as too many threads
    expect(lib.teeny_hip_launch(FAKE, g, (ctypes.c_uint32 * 3)(65536, 65536, 1), 0, None, None),
           _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_hip_launch(FAKE, g, (ctypes.c_uint32 * 3)(1024, 1024, 4096), 0, None, None),
           _lib.ERR_INVALID_ARGUMENT)


def test_example_code_object_built():
    # the stand-alone gfx950 code object the module surface loads (hipcc --genco)
    assert os.path.exists(_lib.EXAMPLE_MODULE_PATH)
    with open(_lib.EXAMPLE_MODULE_PATH, "rb") as f:
        assert f.read(4) == b"\x7fELF"


def test_dispatch_new_names_errors():
    d = lib.teeny_dispatch
    grid = (ctypes.c_uint32 * 3)(8, 4, 1)
    attn = packed(*([(_lib.ARG_PTR, FAKE)] * 5 + [(_lib.ARG_I32, 8), (_lib.ARG_I32, 8), (_lib.ARG_F32, 0.125),
                                                  (_lib.ARG_F32, float("-inf"))]))
    # multi_head_attention: four const generics; grid[1] a multiple of Q_HEADS; heads divide
    expect(d(b"multi_head_attention_forward_entry_point", (ctypes.c_int64 * 2)(64, 1), 2, attn, 9, grid,
             _lib.BF16, None), _lib.ERR_INVALID_ARGUMENT)
    expect(d(b"multi_head_attention_forward_entry_point", (ctypes.c_int64 * 4)(64, 1, 3, 1), 4, attn, 9, grid,
             _lib.BF16, None), _lib.ERR_SHAPE_MISMATCH)
    expect(d(b"multi_head_attention_forward_entry_point", (ctypes.c_int64 * 4)(64, 1, 4, 3), 4, attn, 9, grid,
             _lib.BF16, None), _lib.ERR_SHAPE_MISMATCH)
    expect(d(b"flash_attention2_forward_entry_point", (ctypes.c_int64 * 3)(64, 1, 0), 3, attn, 9, grid,
             _lib.BF16, None), _lib.ERR_INVALID_ARGUMENT)
    # w8a16: bf16 only, USE_BIAS/ACT const generics
    lin = packed(*([(_lib.ARG_PTR, FAKE)] * 5 + [(_lib.ARG_I32, 16)] * 3))
    expect(d(b"w8a16_linear_forward_entry_point", (ctypes.c_int64 * 2)(0, 0), 2, lin, 8, grid, _lib.F32, None),
           _lib.ERR_UNSUPPORTED_DTYPE)
    expect(d(b"w8a16_linear_forward_entry_point", (ctypes.c_int64 * 1)(0), 1, lin, 8, grid, _lib.BF16, None),
           _lib.ERR_INVALID_ARGUMENT)
    # quantize: dims must be i64 arguments, as many as ndim says
    q = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE),
               (_lib.ARG_PTR, None), (_lib.ARG_I32, 2), (_lib.ARG_I32, 4), (_lib.ARG_I32, 4))
    cg = (ctypes.c_int64 * 5)(1, 0, 1, 1, 8)
    expect(d(b"quantize_affine_entry_point", cg, 5, q, 8, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    q_short = packed((_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE), (_lib.ARG_PTR, FAKE),
                     (_lib.ARG_PTR, None), (_lib.ARG_I32, 2))
    expect(d(b"quantize_affine_entry_point", cg, 5, q_short, 6, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)
    expect(d(b"dequantize_affine_entry_point", cg, 5, q, 8, grid, _lib.F32, None), _lib.ERR_INVALID_ARGUMENT)


def test_attention_forward_errors():
    f = lib.teeny_attention_forward
    # q_heads must be a multiple of kv_heads; sizes non-negative
    expect(f(FAKE, FAKE, FAKE, FAKE, None, 2, 6, 4, 16, 16, 64, 0.125, 0, _lib.BF16, None), _lib.ERR_SHAPE_MISMATCH)
    expect(f(FAKE, FAKE, FAKE, FAKE, None, -1, 4, 4, 16, 16, 64, 0.125, 0, _lib.BF16, None), _lib.ERR_SHAPE_MISMATCH)
    expect(f(FAKE, None, FAKE, FAKE, None, 2, 4, 2, 16, 16, 64, 0.125, 1, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    expect(f(FAKE, FAKE, FAKE, FAKE, None, 2, 4, 2, 16, 16, 96, 0.125, 1, _lib.BF16, None), _lib.ERR_UNSUPPORTED)
    expect(f(FAKE_ODD, FAKE, FAKE, FAKE, None, 2, 4, 2, 16, 16, 64, 0.125, 1, _lib.BF16, None), _lib.ERR_MISALIGNED)
    assert f(None, None, None, None, None, 0, 4, 2, 16, 16, 64, 0.125, 1, _lib.BF16, None) == _lib.OK


def test_graph_capture_errors():
    g = ctypes.c_void_p()
    expect(lib.teeny_hip_stream_begin_capture(None), _lib.ERR_INVALID_ARGUMENT)
    expect(lib.teeny_hip_stream_end_capture(None, ctypes.byref(g)), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_stream_end_capture(FAKE, None), _lib.ERR_NULL_POINTER)
    expect(lib.teeny_hip_graph_launch(None, None), _lib.ERR_NULL_POINTER)
    assert lib.teeny_hip_graph_destroy(None) == _lib.OK


def test_training_kernel_errors():
    lf = lib.teeny_layer_norm_forward
    expect(lf(FAKE, FAKE, FAKE, FAKE, None, FAKE, 4, 8, 1e-5, _lib.F32, None), _lib.ERR_NULL_POINTER)
    lb = lib.teeny_layer_norm_backward
    expect(lb(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, None, 4, 8, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(lb(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 0, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(lb(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, -1, 8, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(lb(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, FAKE, 4, 8, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    assert lb(None, None, None, None, None, None, None, None, 0, 8, _lib.F32, None) == _lib.OK
    rb = lib.teeny_rms_norm_backward
    expect(rb(FAKE, FAKE, FAKE, None, None, FAKE, 4, 8, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    size = ctypes.c_size_t(123)
    assert lib.teeny_norm_backward_workspace_size(100, 4096, 0, _lib.BF16, ctypes.byref(size)) == _lib.OK
    assert size.value > 0 and size.value % (4096 * 4) == 0
    assert lib.teeny_norm_backward_workspace_size(100, 4095, 1, _lib.BF16, ctypes.byref(size)) == _lib.OK
    assert size.value == 0  # no register plan for a ragged row: no scratch either
    expect(lib.teeny_norm_backward_workspace_size(1, 8, 0, _lib.F32, None), _lib.ERR_NULL_POINTER)

    cbx, cbw, cb = lib.teeny_conv2d_backward_dx, lib.teeny_conv2d_backward_dw, lib.teeny_conv2d_backward
    expect(cbx(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 7, 8, conv_params(), _lib.F32, _lib.NCHW, None),
           _lib.ERR_SHAPE_MISMATCH)
    expect(cbx(None, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, _lib.NCHW, None),
           _lib.ERR_NULL_POINTER)
    expect(cbw(FAKE, None, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, _lib.NCHW, None),
           _lib.ERR_NULL_POINTER)
    expect(cb(FAKE, FAKE, None, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, _lib.NHWC, None),
           _lib.ERR_NULL_POINTER)
    expect(cbw(FAKE, FAKE, FAKE, 1, 4, 4, 8, 8, 8, 8, conv_params(), _lib.I8, _lib.NCHW, None),
           _lib.ERR_UNSUPPORTED_DTYPE)
    # an empty batch: nothing to write for dx (dw would be zero-filled on a device)
    assert cbx(None, None, FAKE, 0, 4, 4, 8, 8, 8, 8, conv_params(), _lib.F32, _lib.NCHW, None) == _lib.OK
    assert lib.teeny_conv2d_backward_workspace_size(2, 64, 128, 14, 14, 14, 14, conv_params(), _lib.BF16,
                                                    _lib.NHWC, ctypes.byref(size)) == _lib.OK
    assert size.value >= 128 * 9 * 64 * 2  # the flipped weights at least
    assert lib.teeny_conv2d_backward_workspace_size(2, 64, 128, 14, 14, 14, 14, conv_params(), _lib.F32,
                                                    _lib.NCHW, ctypes.byref(size)) == _lib.OK
    assert size.value == 0


def test_attention_backward_errors():
    dq, dkv = lib.teeny_flash_attention2_backward_dq, lib.teeny_flash_attention2_backward_dkv
    ab = lib.teeny_attention_backward
    args6 = (FAKE,) * 6
    expect(dq(*args6, None, 8, 8, 0.125, 4, 64, 0, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(dq(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 8, 8, 0.125, 4, 64, 0, _lib.F32, None),
           _lib.ERR_NULL_POINTER)
    expect(dkv(*args6, FAKE, None, 8, 8, 0.125, 4, 64, 0, _lib.F32, None), _lib.ERR_NULL_POINTER)
    expect(dq(*args6, FAKE, 8, 8, 0.125, 4, 48, 0, _lib.F32, None), _lib.ERR_UNSUPPORTED)
    expect(dq(*args6, FAKE, 8, 8, 0.125, 4, 64, 0, _lib.I8, None), _lib.ERR_UNSUPPORTED_DTYPE)
    expect(dq(*args6, FAKE, 8, 0, 0.125, 4, 64, 0, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(dq(*args6, FAKE, -1, 8, 0.125, 4, 64, 0, _lib.F32, None), _lib.ERR_SHAPE_MISMATCH)
    expect(ab(*args6, FAKE, FAKE, FAKE, 2, 6, 4, 8, 8, 64, 0.125, 0, _lib.BF16, None), _lib.ERR_SHAPE_MISMATCH)
    expect(ab(*args6, FAKE, None, FAKE, 2, 4, 2, 8, 8, 64, 0.125, 0, _lib.BF16, None), _lib.ERR_NULL_POINTER)
    assert ab(*args6, FAKE, FAKE, FAKE, 0, 4, 2, 8, 8, 64, 0.125, 0, _lib.BF16, None) == _lib.OK
    size = ctypes.c_size_t(0)
    assert lib.teeny_attention_backward_workspace_size(2, 8, 1000, ctypes.byref(size)) == _lib.OK
    assert size.value == 2 * 8 * 1000 * 4
    expect(lib.teeny_attention_backward_workspace_size(2, 8, 10, None), _lib.ERR_NULL_POINTER)
    # the backward's own limits (B*H <= 65535, n_ctx_q < 2^31) bound the size:
    # no wrapped products
    expect(lib.teeny_attention_backward_workspace_size(2 ** 40, 2 ** 30, 2 ** 20, ctypes.byref(size)),
           _lib.ERR_SHAPE_MISMATCH)
    expect(lib.teeny_attention_backward_workspace_size(256, 256, 8, ctypes.byref(size)), _lib.ERR_SHAPE_MISMATCH)
    expect(lib.teeny_attention_backward_workspace_size(1, 1, 2 ** 31, ctypes.byref(size)), _lib.ERR_SHAPE_MISMATCH)
    assert lib.teeny_attention_backward_workspace_size(255, 257, 2 ** 31 - 1, ctypes.byref(size)) == _lib.OK
    assert size.value == 255 * 257 * (2 ** 31 - 1) * 4
