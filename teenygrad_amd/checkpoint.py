"""Compressed-tensors int8 checkpoints (teeny-quant's output convention).

Reading goes through the native reader of the C ABI (teeny_checkpoint_*,
csrc/safetensors.cpp + checkpoint.cpp): the file is memory-mapped, its
header validated, and W8A16 layers are copied straight into device buffers
for ``kernels.w8a16_linear`` / ``kernels.w8a16_conv2d``.  Writing mirrors
teeny-quant's quantize path on the GPU quantizer (bit-exact with
quantize_affine).

Reference: utilities/teeny-quant/src/format.rs — naming (foo.weight I8,
foo.weight_scale F32 per group, foo.weight_zero_point I32 when asymmetric,
:16-35, :118-126), quantize_tensor (:145-246), dequantize_tensor
(:249-289), build_config / config_to_metadata (:291-355), should_quantize
(:129-133: rank >= 2 float tensors; the rest pass through and are listed
in ``ignore``); utilities/teeny-quant/src/write.rs (safetensors output).
"""
from __future__ import annotations

import ctypes
import json
import struct
from typing import Dict, Optional, Tuple

import numpy as np

from . import _lib
from ._lib import check, lib
from .dtypes import f32, i8
from .runtime import Buffer, Stream, _h

# safetensors dtype name -> numpy dtype of the raw little-endian elements
# (bf16 as its uint16 bit patterns, like the rest of this package)
NUMPY_OF = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16, "I64": np.int64,
            "I32": np.int32, "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_}
GRAN_NAME = {_lib.PER_TENSOR: "tensor", _lib.PER_CHANNEL: "channel", _lib.GROUP: "group"}


class Checkpoint:
    """A read-only, memory-mapped .safetensors file."""

    def __init__(self, path: Optional[str] = None, image: Optional[bytes] = None):
        h = ctypes.c_void_p()
        if image is not None:
            self._image = ctypes.create_string_buffer(bytes(image), len(image))  # kept alive
            check(lib.teeny_checkpoint_open_image(self._image, len(image), ctypes.byref(h)))
        else:
            check(lib.teeny_checkpoint_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            check(lib.teeny_checkpoint_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self) -> Dict[str, dict]:
        n = ctypes.c_int64()
        check(lib.teeny_checkpoint_num_tensors(self.handle, ctypes.byref(n)))
        out = {}
        for i in range(n.value):
            info = _lib.TensorInfo()
            check(lib.teeny_checkpoint_tensor_info(self.handle, i, ctypes.byref(info)))
            out[info.name.decode()] = {"index": i, "dtype": info.dtype.decode(),
                                       "shape": tuple(info.shape[d] for d in range(info.ndim)),
                                       "nbytes": int(info.nbytes)}
        return out

    def quant_scheme(self) -> Optional[dict]:
        """The quantization_config's scheme, or None if the file has none."""
        q = _lib.QuantScheme()
        check(lib.teeny_checkpoint_quant_scheme(self.handle, ctypes.byref(q)))
        if not q.present:
            return None
        return {"quant_method": q.quant_method.decode(), "format": q.format.decode(), "type": q.type.decode(),
                "num_bits": q.num_bits, "symmetric": bool(q.symmetric),
                "strategy": GRAN_NAME.get(q.granularity, "unknown"), "granularity": q.granularity,
                "axis": q.axis, "group_size": q.group_size, "n_config_groups": q.n_config_groups}

    def _entry(self, name: str) -> dict:
        t = self.tensors().get(name)
        if t is None:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        return t

    def read(self, name: str) -> np.ndarray:
        """Tensor `name` as a host array (bf16 as uint16 bit patterns)."""
        t = self._entry(name)
        arr = np.empty(t["shape"], dtype=NUMPY_OF[t["dtype"]])
        check(lib.teeny_checkpoint_read(self.handle, t["index"], arr.ctypes.data, t["nbytes"], 0, None))
        return arr

    def to_device(self, name: str, dtype, stream: Optional[Stream] = None) -> Buffer:
        """Tensor `name`'s bytes in a new device buffer of `dtype`."""
        t = self._entry(name)
        buf = Buffer(dtype, t["shape"])
        if buf.nbytes != t["nbytes"]:
            raise ValueError(f"{name}: {t['nbytes']} bytes in the file, {buf.nbytes} for {buf.dtype.name}")
        check(lib.teeny_checkpoint_read(self.handle, t["index"], buf.ptr, buf.nbytes, 1, _h(stream)))
        return buf

    def load_w8a16(self, weight_name: str, stream: Optional[Stream] = None) -> Tuple[Buffer, Buffer]:
        """(qweight int8, scale fp32 [N]) on the device, for w8a16_linear
        ([N, K], the file's own shape) or w8a16_conv2d: a rank-4 conv weight
        is stored in the reference's order [C_OUT, C_IN/G, KH, KW] and comes
        back repacked as [C_OUT, KH, KW, C_IN/G]."""
        n, k = ctypes.c_int64(), ctypes.c_int64()
        check(lib.teeny_checkpoint_w8a16_shape(self.handle, weight_name.encode(), ctypes.byref(n), ctypes.byref(k)))
        shape = tuple(self._entry(weight_name)["shape"])
        if len(shape) == 4:
            shape = (shape[0], shape[2], shape[3], shape[1])
        q = Buffer(i8, shape)
        s = Buffer(f32, (n.value,))
        check(lib.teeny_checkpoint_load_w8a16(self.handle, weight_name.encode(), q.ptr, s.ptr, n.value, k.value,
                                              _h(stream)))
        return q, s

    def dequantize(self, weight_name: str, stream: Optional[Stream] = None) -> Buffer:
        """Any int8 scheme (tensor / channel / group, symmetric or not) back to
        fp32 on the device: dequantize_tensor (format.rs:249-289) on the GPU."""
        from .kernels import dequantize_affine
        sch = self.quant_scheme()
        if sch is None or sch["type"] != "int" or sch["num_bits"] != 8 or sch["format"] != "int-quantized":
            raise ValueError(f"{weight_name}: not an 8-bit int-quantized compressed-tensors checkpoint")
        # channel / group strategies must name their axis (and group the
        # group size), as granularity_from_config requires (validate.rs:94-103)
        if sch["strategy"] in ("channel", "group") and sch["axis"] < 0:
            raise ValueError(f"{weight_name}: strategy '{sch['strategy']}' without an axis is ambiguous")
        if sch["strategy"] == "group" and not sch["group_size"]:
            raise ValueError(f"{weight_name}: strategy 'group' without a group_size")
        shape = self._entry(weight_name)["shape"]
        q = self.to_device(weight_name, i8, stream)
        s = self.to_device(weight_name + "_scale", f32, stream)
        z = None if sch["symmetric"] else self.to_device(weight_name + "_zero_point", "i32", stream)
        axis = max(0, sch["axis"])
        gs = sch["group_size"] or 1
        return dequantize_affine(q, s, z, list(shape), sch["strategy"], axis, gs, stream=stream)


# ── writing ─────────────────────────────────────────────────────────────────


def serialize_safetensors(tensors: Dict[str, Tuple[str, tuple, bytes]], metadata: Optional[Dict[str, str]] = None) -> bytes:
    """safetensors bytes: 8-byte header length, JSON header (padded with
    spaces to a multiple of 8), tensor data in name order."""
    header, offset, chunks = {}, 0, []
    if metadata:
        header["__metadata__"] = dict(metadata)
    for name in sorted(tensors):
        dtype, shape, data = tensors[name]
        header[name] = {"dtype": dtype, "shape": [int(d) for d in shape], "data_offsets": [offset, offset + len(data)]}
        chunks.append(data)
        offset += len(data)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(chunks)


def build_config(granularity: str, axis: int, group_size: int, symmetric: bool, ignore) -> dict:
    """teeny-quant's quantization_config for an int8 scheme (format.rs:291-341)."""
    weights = {"num_bits": 8, "type": "int", "symmetric": bool(symmetric), "strategy": granularity}
    if granularity in ("channel", "group"):
        weights["axis"] = int(axis)
    if granularity == "group":
        weights["group_size"] = int(group_size)
    cfg = {"quant_method": "compressed-tensors", "format": "int-quantized",
           "config_groups": {"group_0": {"weights": weights, "targets": ["*"]}}}
    if ignore:
        cfg["ignore"] = list(ignore)
    return cfg


def quantize_checkpoint(tensors: Dict[str, np.ndarray], granularity: str = "channel", axis: int = 0,
                        group_size: int = 1, symmetric: bool = True, stream: Optional[Stream] = None) -> bytes:
    """Quantizes every rank >= 2 fp32 tensor to int8 on the GPU (bit-exact
    with teeny-quant's quantize_affine) and returns the compressed-tensors
    .safetensors bytes; rank < 2 tensors pass through unchanged and are
    listed in ``ignore`` (format.rs:129-133, :145-246)."""
    from .kernels import quantize_affine
    from .runtime import Buffer as _B
    out, ignore = {}, []
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr)
        if arr.ndim < 2 or arr.dtype != np.float32:
            dt = {v: k for k, v in NUMPY_OF.items()}[arr.dtype.type]
            out[name] = (dt, arr.shape, arr.tobytes())
            ignore.append(name)
            continue
        d = _B(f32, (arr.size,)).to_device(arr.reshape(-1), stream)
        q, s, z, _ = quantize_affine(d, list(arr.shape), granularity, axis, group_size, symmetric, 8, stream=stream)
        out[name] = ("I8", arr.shape, q.to_host(stream).tobytes())
        out[name + "_scale"] = ("F32", (s.numel,), s.to_host(stream).tobytes())
        if not symmetric:
            out[name + "_zero_point"] = ("I32", (z.numel,), z.to_host(stream).tobytes())
    cfg = build_config(granularity, axis, group_size, symmetric, sorted(ignore))
    return serialize_safetensors(out, {"quantization_config": json.dumps(cfg, separators=(",", ":"))})
