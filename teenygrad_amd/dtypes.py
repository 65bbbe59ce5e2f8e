"""Element types of the C ABI and their host (numpy) representations.

bfloat16 has no numpy dtype; host-side bf16 tensors are ``uint16`` arrays of
IEEE bfloat16 bit patterns.  ``to_bf16`` rounds fp32 to nearest-even (NaN
stays a quiet NaN), which is what the GPU's v_cvt_pk_bf16_f32 does, so a
host-rounded input and a device-rounded output use the same rounding.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib


@dataclass(frozen=True)
class DType:
    name: str
    code: int
    host: type
    itemsize: int


f32 = DType("f32", _lib.F32, np.float32, 4)
bf16 = DType("bf16", _lib.BF16, np.uint16, 2)
i8 = DType("i8", _lib.I8, np.int8, 1)
i32 = DType("i32", -1, np.int32, 4)
u32 = DType("u32", -1, np.uint32, 4)

_BY_NAME = {d.name: d for d in (f32, bf16, i8, i32, u32)}
_BY_HOST = {np.dtype(np.float32): f32, np.dtype(np.uint16): bf16, np.dtype(np.int8): i8,
            np.dtype(np.int32): i32, np.dtype(np.uint32): u32}


def from_any(d) -> DType:
    if isinstance(d, DType):
        return d
    if isinstance(d, str):
        return _BY_NAME[d]
    return _BY_HOST[np.dtype(d)]


def to_bf16(a) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    # uint32 is wide enough: only NaN bit patterns can carry past 2^32, and
    # NaNs are rewritten below
    r = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = ((a.view(np.uint32)[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def from_bf16(b) -> np.ndarray:
    """bf16 bit patterns -> fp32 (exact)."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """fp32 values rounded to the nearest bf16, returned as fp32."""
    return from_bf16(to_bf16(a))
