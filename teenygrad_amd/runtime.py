"""Device, buffer, stream and event objects over the teeny_hip C ABI.

Mirrors the reference's runtime façade and CUDA driver surface:
``teeny_runtime::open()`` (runtime/teeny-runtime/src/lib.rs:250-259),
``device.buffer::<T>(n)`` / ``to_device`` / ``to_host``
(drivers/teeny-cuda/src/device/buffer.rs:37-62) and event timing
(drivers/teeny-cuda/src/model/mod.rs:1729-1797).  Host data is numpy;
bfloat16 host arrays are ``uint16`` bit patterns (see ``dtypes``).
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import check, lib
from .dtypes import DType, from_any

__all__ = ["open", "Device", "Buffer", "Stream", "Event", "Graph", "device_count"]


def device_count() -> int:
    n = ctypes.c_int32(0)
    check(lib.teeny_hip_device_count(ctypes.byref(n)))
    return n.value


class Stream:
    """A HIP stream at the default priority (``None`` handle = null stream)."""

    def __init__(self, handle: Optional[int] = None, owned: bool = False):
        self.handle = handle
        self._owned = owned
        self._workspace = None

    @classmethod
    def create(cls) -> "Stream":
        h = ctypes.c_void_p()
        check(lib.teeny_hip_stream_create(ctypes.byref(h)))
        return cls(h.value, owned=True)

    def synchronize(self) -> None:
        check(lib.teeny_hip_stream_sync(self.handle))

    def set_workspace(self, buf: Optional["Buffer"]) -> None:
        """Attaches ``buf`` (caller-owned, kept alive here while attached) as
        operator scratch for work on this stream; ``None`` detaches."""
        if buf is None:
            check(lib.teeny_hip_stream_set_workspace(self.handle, None, 0))
        else:
            check(lib.teeny_hip_stream_set_workspace(self.handle, buf.ptr, buf.nbytes))
        self._workspace = buf

    def begin_capture(self) -> None:
        """Record the work enqueued on this stream until end_capture()."""
        check(lib.teeny_hip_stream_begin_capture(self.handle))

    def end_capture(self) -> "Graph":
        g = ctypes.c_void_p()
        check(lib.teeny_hip_stream_end_capture(self.handle, ctypes.byref(g)))
        return Graph(g.value)

    def destroy(self) -> None:
        if self._owned and self.handle:
            check(lib.teeny_hip_stream_destroy(self.handle))
        self.handle = None
        self._owned = False

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


NULL_STREAM = Stream(None)


def _h(stream: Optional[Stream]):
    return None if stream is None else stream.handle


class Graph:
    """An instantiated HIP graph from Stream.begin_capture()/end_capture()."""

    def __init__(self, handle: int):
        self.handle = handle

    def launch(self, stream: Optional["Stream"] = None) -> None:
        check(lib.teeny_hip_graph_launch(self.handle, _h(stream)))

    def destroy(self) -> None:
        if self.handle:
            check(lib.teeny_hip_graph_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        check(lib.teeny_hip_event_create(ctypes.byref(h)))
        self.handle = h.value

    def record(self, stream: Optional[Stream] = None) -> None:
        check(lib.teeny_hip_event_record(self.handle, _h(stream)))

    def synchronize(self) -> None:
        check(lib.teeny_hip_event_sync(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib.teeny_hip_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib.teeny_hip_event_destroy(self.handle)
        except Exception:
            pass


class Buffer:
    """A device allocation with a dtype and a logical shape."""

    def __init__(self, dtype, shape: Sequence[int]):
        self.dtype: DType = from_any(dtype)
        self.shape = tuple(int(s) for s in shape)
        self.numel = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.numel * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(lib.teeny_hip_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @property
    def handle(self):
        return self.ptr

    def to_device(self, host: np.ndarray, stream: Optional[Stream] = None) -> "Buffer":
        arr = np.ascontiguousarray(host, dtype=self.dtype.host)
        if arr.size != self.numel:
            raise ValueError(f"host array has {arr.size} elements, buffer {self.numel}")
        check(lib.teeny_hip_memcpy_h2d(self.ptr, arr.ctypes.data, self.nbytes, _h(stream)))
        return self

    def to_host(self, stream: Optional[Stream] = None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype.host)
        check(lib.teeny_hip_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, _h(stream)))
        return out

    def zero_(self, stream: Optional[Stream] = None) -> "Buffer":
        check(lib.teeny_hip_memset(self.ptr, 0, self.nbytes, _h(stream)))
        return self

    def free(self) -> None:
        if self.ptr:
            check(lib.teeny_hip_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"Buffer({self.dtype.name}, {self.shape}, ptr=0x{self.ptr or 0:x})"


class Device:
    """An opened HIP device (teeny_runtime::open equivalent)."""

    def __init__(self, ordinal: int = 0):
        self.ordinal = ordinal
        check(lib.teeny_hip_device_open(ordinal))

    def info(self) -> dict:
        info = _lib.DeviceInfo()
        check(lib.teeny_hip_device_info(self.ordinal, ctypes.byref(info)))
        return {
            "name": info.name.decode(),
            "arch": info.arch.decode(),
            "compute_units": info.compute_units,
            "wavefront_size": info.wavefront_size,
            "clock_khz": info.clock_khz,
            "memory_clock_khz": info.memory_clock_khz,
            "memory_bus_width": info.memory_bus_width,
            "l2_cache_bytes": info.l2_cache_bytes,
            "total_global_mem": info.total_global_mem,
            "shared_mem_per_block": info.shared_mem_per_block,
        }

    def buffer(self, dtype, shape) -> Buffer:
        if isinstance(shape, int):
            shape = (shape,)
        return Buffer(dtype, shape)

    def upload(self, host: np.ndarray, dtype=None) -> Buffer:
        dt = from_any(dtype) if dtype is not None else from_any(host.dtype)
        return Buffer(dt, host.shape).to_device(host)

    def synchronize(self) -> None:
        check(lib.teeny_hip_device_synchronize())


def open(ordinal: int = 0) -> Device:  # noqa: A001 - mirrors teeny_runtime::open
    return Device(ordinal)
