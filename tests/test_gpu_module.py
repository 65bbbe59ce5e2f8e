"""GPU: the code-object surface of the C ABI — module load (from a path and
from an in-memory image), function lookup, and a raw launch with a void**
argument array, the shape of the reference's CudaArgPacker
(drivers/teeny-cuda/src/device/program.rs:327-390, device/mod.rs:49-110,
:430-490).  The code object is csrc/module_example.hip built by hipcc --genco:
y = a * x + y."""
import ctypes

import numpy as np
import pytest

import teenygrad_amd as tg
from teenygrad_amd import _lib
from teenygrad_amd._lib import check, lib

pytestmark = pytest.mark.gpu


def launch_axpy(fn, a, xb, yb, n, grid, block, stream=None):
    ca, cx, cy, cn = ctypes.c_float(a), ctypes.c_void_p(xb.ptr), ctypes.c_void_p(yb.ptr), ctypes.c_int32(n)
    args = (ctypes.c_void_p * 4)(*(ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in (ca, cx, cy, cn)))
    g = (ctypes.c_uint32 * 3)(*grid)
    b = (ctypes.c_uint32 * 3)(*block)
    check(lib.teeny_hip_launch(fn, g, b, 0, stream.handle if stream else None, args))


@pytest.mark.parametrize("how", ["path", "image"])
def test_module_load_and_launch(dev, how):
    print(f"[module] load from {how}", flush=True)
    mod = ctypes.c_void_p()
    if how == "path":
        check(lib.teeny_hip_module_load(ctypes.byref(mod), _lib.EXAMPLE_MODULE_PATH.encode()))
    else:
        image = open(_lib.EXAMPLE_MODULE_PATH, "rb").read()
        buf = ctypes.create_string_buffer(image, len(image))
        check(lib.teeny_hip_module_load_data(ctypes.byref(mod), buf))
    try:
        fn = ctypes.c_void_p()
        check(lib.teeny_hip_module_get_function(ctypes.byref(fn), mod, b"teeny_example_axpy"))
        missing = ctypes.c_void_p()
        assert lib.teeny_hip_module_get_function(ctypes.byref(missing), mod, b"no_such_kernel") == _lib.ERR_NOT_FOUND
        rng = np.random.default_rng(11)
        n = 100_003
        x = rng.standard_normal(n, dtype=np.float32)
        y = rng.standard_normal(n, dtype=np.float32)
        xb, yb = dev.upload(x), dev.upload(y)
        stream = tg.Stream.create()
        # a grid smaller than n / block: the kernel's grid-stride loop covers the rest
        launch_axpy(fn, 2.5, xb, yb, n, (97, 1, 1), (256, 1, 1), stream)
        stream.synchronize()
        # the compiler may contract a * x + y into one fused multiply-add: the
        # result is the float32 rounding of the exact value (within an ulp)
        y1 = yb.to_host()
        want = 2.5 * x.astype(np.float64) + y
        np.testing.assert_allclose(y1, want, rtol=1.2e-7, atol=1e-30)
        launch_axpy(fn, -1.0, xb, yb, n, (1, 1, 1), (64, 1, 1))
        dev.synchronize()
        np.testing.assert_array_equal(yb.to_host(), y1 - x)  # a = -1: exact
        stream.destroy()
    finally:
        check(lib.teeny_hip_module_unload(mod))
