"""ctypes binding of libteeny_hip.so (the C ABI declared in include/teeny_hip.h).

The shared library is built in-tree (``make -C teenygrad_amd/csrc`` or
``__graft_entry__.build()``) next to this file.  Importing this module when
the library is missing raises immediately: there is no fallback
implementation of any operator.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint32, c_void_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libteeny_hip.so")
# A stand-alone gfx950 code object (csrc/module_example.hip, built with
# `hipcc --genco`) that the module-load / raw-launch surface can load.
EXAMPLE_MODULE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "teeny_example.hsaco")

# status codes (include/teeny_hip.h)
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_NULL_POINTER = 2
ERR_UNSUPPORTED_DTYPE = 3
ERR_SHAPE_MISMATCH = 4
ERR_MISALIGNED = 5
ERR_INVALID_AXIS = 6
ERR_INVALID_GROUP_SIZE = 7
ERR_NO_DEVICE = 8
ERR_HIP = 9
ERR_NOT_FOUND = 10
ERR_UNSUPPORTED = 11

# dtypes / layouts / activations / granularities / argument kinds
F32, BF16, I8 = 0, 1, 2
NCHW, NHWC = 0, 1
ACT_NONE, ACT_RELU, ACT_GELU_TANH, ACT_SILU = 0, 1, 2, 3
PER_TENSOR, PER_CHANNEL, GROUP = 0, 1, 2
PW_RELU, PW_GELU_TANH, PW_SILU, PW_SIGMOID, PW_TANH = 1, 2, 3, 4, 5
ARG_PTR, ARG_I32, ARG_I64, ARG_F32, ARG_F64, ARG_U32, ARG_BOOL = range(7)


class TeenyError(RuntimeError):
    """A non-zero teeny_status, with the library's message."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", c_int32),
        ("wavefront_size", c_int32),
        ("clock_khz", c_int32),
        ("memory_clock_khz", c_int32),
        ("memory_bus_width", c_int32),
        ("l2_cache_bytes", c_int32),
        ("total_global_mem", c_int64),
        ("shared_mem_per_block", c_int64),
    ]


class Conv2dParams(ctypes.Structure):
    _fields_ = [
        ("KH", c_int32), ("KW", c_int32),
        ("stride_h", c_int32), ("stride_w", c_int32),
        ("pad_h", c_int32), ("pad_w", c_int32),
        ("groups", c_int32), ("act", c_int32),
    ]


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_char * 16), ("ndim", c_int32),
                ("pad_", c_int32), ("shape", c_int64 * 8), ("nbytes", ctypes.c_uint64)]


class QuantScheme(ctypes.Structure):
    _fields_ = [("present", c_int32), ("num_bits", c_int32), ("symmetric", c_int32),
                ("granularity", c_int32), ("axis", c_int64), ("group_size", c_int64),
                ("n_config_groups", c_int32), ("quant_method", ctypes.c_char * 64),
                ("format", ctypes.c_char * 64), ("type", ctypes.c_char * 16)]


class _ArgValue(ctypes.Union):
    _fields_ = [("ptr", c_void_p), ("i32", c_int32), ("i64", c_int64), ("f32", c_float),
                ("f64", ctypes.c_double), ("u32", c_uint32), ("b", c_int32)]


class TeenyArg(ctypes.Structure):
    _fields_ = [("kind", c_int32), ("pad_", c_int32), ("v", _ArgValue)]


S = c_int32  # teeny_status
P = c_void_p
_SIGS = {
    "teeny_hip_last_error": (c_char_p, []),
    "teeny_status_string": (c_char_p, [S]),
    "teeny_hip_version": (c_char_p, []),
    "teeny_hip_init": (S, []),
    "teeny_hip_device_count": (S, [POINTER(c_int32)]),
    "teeny_hip_device_open": (S, [c_int32]),
    "teeny_hip_device_info": (S, [c_int32, POINTER(DeviceInfo)]),
    "teeny_hip_device_synchronize": (S, []),
    "teeny_hip_device_close": (S, [c_int32]),
    "teeny_hip_malloc": (S, [POINTER(c_void_p), c_size_t]),
    "teeny_hip_free": (S, [P]),
    "teeny_hip_memcpy_h2d": (S, [P, P, c_size_t, P]),
    "teeny_hip_memcpy_d2h": (S, [P, P, c_size_t, P]),
    "teeny_hip_memcpy_d2d": (S, [P, P, c_size_t, P]),
    "teeny_hip_memset": (S, [P, c_int32, c_size_t, P]),
    "teeny_hip_stream_create": (S, [POINTER(c_void_p)]),
    "teeny_hip_stream_destroy": (S, [P]),
    "teeny_hip_stream_sync": (S, [P]),
    "teeny_hip_stream_set_workspace": (S, [P, P, c_size_t]),
    "teeny_hip_stream_begin_capture": (S, [P]),
    "teeny_hip_stream_end_capture": (S, [P, POINTER(c_void_p)]),
    "teeny_hip_graph_launch": (S, [P, P]),
    "teeny_hip_graph_destroy": (S, [P]),
    "teeny_hip_event_create": (S, [POINTER(c_void_p)]),
    "teeny_hip_event_destroy": (S, [P]),
    "teeny_hip_event_record": (S, [P, P]),
    "teeny_hip_event_sync": (S, [P]),
    "teeny_hip_event_elapsed_ms": (S, [POINTER(c_float), P, P]),
    "teeny_hip_module_load": (S, [POINTER(c_void_p), c_char_p]),
    "teeny_hip_module_load_data": (S, [POINTER(c_void_p), P]),
    "teeny_hip_module_get_function": (S, [POINTER(c_void_p), P, c_char_p]),
    "teeny_hip_module_unload": (S, [P]),
    "teeny_hip_launch": (S, [P, POINTER(c_uint32), POINTER(c_uint32), c_uint32, P, POINTER(c_void_p)]),
    "teeny_relu_forward": (S, [P, P, c_int64, c_int32, P]),
    "teeny_gelu_forward": (S, [P, P, c_int64, c_int32, P]),
    "teeny_silu_forward": (S, [P, P, c_int64, c_int32, P]),
    "teeny_relu_backward": (S, [P, P, P, c_int64, c_int32, P]),
    "teeny_gelu_backward": (S, [P, P, P, c_int64, c_int32, P]),
    "teeny_silu_backward": (S, [P, P, P, c_int64, c_int32, P]),
    "teeny_layer_norm_forward_inference": (S, [P, P, P, P, c_int64, c_int64, c_float, c_int32, P]),
    "teeny_rms_norm_forward": (S, [P, P, P, P, c_int64, c_int64, c_float, c_int32, P]),
    "teeny_layer_norm_forward": (S, [P, P, P, P, P, P, c_int64, c_int64, c_float, c_int32, P]),
    "teeny_layer_norm_backward": (S, [P, P, P, P, P, P, P, P, c_int64, c_int64, c_int32, P]),
    "teeny_rms_norm_backward": (S, [P, P, P, P, P, P, c_int64, c_int64, c_int32, P]),
    "teeny_norm_backward_workspace_size": (S, [c_int64, c_int64, c_int32, c_int32, POINTER(c_size_t)]),
    "teeny_conv2d_backward_dx": (S, [P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_conv2d_backward_dw": (S, [P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_conv2d_backward": (S, [P, P, P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_conv2d_backward_workspace_size": (S, [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, POINTER(c_size_t)]),
    "teeny_norm_act_forward": (S, [P, P, P, P, c_int64, c_int64, c_float, c_int32, c_int32, c_int32, P]),
    "teeny_conv2d_forward": (S, [P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_conv2d_bias_forward": (S, [P, P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_conv2d_bias_forward_noalloc": (S, [P, P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_flash_attention2_forward": (S, [P, P, P, P, P, c_int64, c_int64, c_float, c_int64, c_int64, c_int32, c_int32, P]),
    "teeny_attention_forward": (S, [P, P, P, P, P] + [c_int64] * 6 + [c_float, c_int32, c_int32, P]),
    "teeny_pointwise_chain_forward": (S, [P, P, POINTER(c_void_p), POINTER(c_int32), c_int32, c_int64, c_int32, P]),
    "teeny_pointwise_chain_backward": (S, [P, P, P, POINTER(c_void_p), POINTER(c_int32), c_int32, c_int64, c_int32,
                                           P]),
    "teeny_conv2d_bn_act_forward": (S, [P, P, P, P, P] + [c_int64] * 7 + [POINTER(c_int64), POINTER(Conv2dParams), c_int32, c_int32, P]),
    "teeny_flash_attention2_backward_dq": (S, [P] * 7 + [c_int64, c_int64, c_float, c_int64, c_int64, c_int32, c_int32, P]),
    "teeny_flash_attention2_backward_dkv": (S, [P] * 8 + [c_int64, c_int64, c_float, c_int64, c_int64, c_int32, c_int32, P]),
    "teeny_attention_backward": (S, [P] * 9 + [c_int64] * 6 + [c_float, c_int32, c_int32, P]),
    "teeny_attention_backward_workspace_size": (S, [c_int64, c_int64, c_int64, POINTER(c_size_t)]),
    "teeny_quant_num_groups": (S, [POINTER(c_int64), c_int32, c_int32, c_int32, c_int64, POINTER(c_int64)]),
    "teeny_quantize_affine": (S, [P, POINTER(c_int64), c_int32, c_int32, c_int32, c_int64, c_int32, c_int32, P, P, P, P, P]),
    "teeny_dequantize_affine": (S, [P, P, P, POINTER(c_int64), c_int32, c_int32, c_int32, c_int64, P, P]),
    "teeny_linear_forward": (S, [P, P, P, P] + [c_int64] * 9 + [c_int32, P]),
    "teeny_w8a16_linear_forward": (S, [P, P, P, P, P, c_int64, c_int64, c_int64, c_int32, P]),
    "teeny_linear_workspace_size": (S, [c_int64, c_int64, c_int64, c_int32, POINTER(c_size_t)]),
    "teeny_linear_backward": (S, [P] * 6 + [c_int64] * 14 + [c_int32, P]),
    "teeny_linear_backward_workspace_size": (S, [c_int64, c_int64, c_int64, c_int32, POINTER(c_size_t)]),
    "teeny_conv2d_workspace_size": (S, [c_int64] * 7 + [POINTER(Conv2dParams), c_int32, c_int32, POINTER(c_size_t)]),
    "teeny_w8a16_conv2d_forward": (S, [P, P, P, P, P] + [c_int64] * 7 + [POINTER(Conv2dParams), P]),
    "teeny_checkpoint_open": (S, [c_char_p, POINTER(c_void_p)]),
    "teeny_checkpoint_open_image": (S, [P, c_size_t, POINTER(c_void_p)]),
    "teeny_checkpoint_close": (S, [P]),
    "teeny_checkpoint_num_tensors": (S, [P, POINTER(c_int64)]),
    "teeny_checkpoint_tensor_info": (S, [P, c_int64, POINTER(TensorInfo)]),
    "teeny_checkpoint_find": (S, [P, c_char_p, POINTER(c_int64)]),
    "teeny_checkpoint_quant_scheme": (S, [P, POINTER(QuantScheme)]),
    "teeny_checkpoint_read": (S, [P, c_int64, P, c_size_t, c_int32, P]),
    "teeny_checkpoint_w8a16_shape": (S, [P, c_char_p, POINTER(c_int64), POINTER(c_int64)]),
    "teeny_checkpoint_load_w8a16": (S, [P, c_char_p, P, P, c_int64, c_int64, P]),
    "teeny_dispatch": (S, [c_char_p, POINTER(c_int64), c_int32, POINTER(TeenyArg), c_int32, POINTER(c_uint32), c_int32, P]),
}

EXPORTED = tuple(_SIGS)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()' or make -C teenygrad_amd/csrc)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def last_error() -> str:
    return lib.teeny_hip_last_error().decode()


def check(status: int) -> None:
    """Raise TeenyError for a non-zero status."""
    if status != OK:
        raise TeenyError(status, last_error())
