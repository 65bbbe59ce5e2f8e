"""teenygrad_amd — MI355X (gfx950) HIP implementation of teeny-kernels' forward
operators (conv2d, flash attention, LayerNorm/RMSNorm, ReLU/GELU/SiLU) and
teeny-quant's int8 affine quantization with W8A16 linear and conv.

The compute lives in libteeny_hip.so (C ABI: include/teeny_hip.h); this
package is the host-side mirror of the reference's runtime and RuntimeOp
contract.  Importing it without the built library raises ImportError.
"""
from . import _lib, dtypes, kernels, runtime, synthetic
from ._lib import TeenyError, check
from .dtypes import bf16, f32, from_bf16, i8, round_bf16, to_bf16
from .runtime import Buffer, Device, Event, Graph, Stream, device_count, open

__all__ = [
    "Buffer", "Device", "Event", "Graph", "Stream", "TeenyError", "bf16", "check", "device_count",
    "dtypes", "f32", "from_bf16", "i8", "kernels", "open", "round_bf16", "runtime",
    "synthetic", "to_bf16",
]
