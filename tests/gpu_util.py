"""Tolerances shared by the GPU parity tests.

fp32 ops: the north-star bound is 1e-5 relative.  Element-wise relative
error is meaningless at values near zero, so fp32 checks use the norm-wise
relative error ||got - ref||_inf / ||ref||_inf <= 1e-5, or an element-wise
relative bound with an absolute floor where stated.

bf16 ops: the bound is 2e-2 absolute after fp32 accumulation.  The kernels
round their fp32 result to bf16 on the store, which alone moves a value by
up to half a bf16 ulp (2^-8 |y|), more than 2e-2 once |y| >= 8, and lands
on the other side of a rounding boundary from the oracle whenever the two
fp32 results straddle one.  So bf16 outputs are checked against the fp32
oracle (unrounded) with |got - ref| <= 2e-2 + 2^-8 |ref|.
"""
import contextlib

import numpy as np

from teenygrad_amd.dtypes import from_bf16

BF16_ATOL = 2e-2
F32_REL = 1e-5


def bf16_bound(ref):
    return BF16_ATOL + np.abs(ref) * 2.0 ** -8


def check_bf16(got_bits, ref32, what=""):
    got = from_bf16(got_bits).astype(np.float64).reshape(-1)
    ref = np.asarray(ref32, dtype=np.float64).reshape(-1)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bad = err > bf16_bound(ref)
    if bad.any():
        i = int(np.argmax(err - bf16_bound(ref)))
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} out of bound; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} err {err[i]:.3g}")
    return float(err.max())


def check_bf16_normwise(got_bits, ref32, what="", rel=8e-3):
    """bf16 output against the fp32 oracle, norm-wise: ||got - ref||_inf <=
    rel * ||ref||_inf (8e-3 is two bf16 ulps of the largest value), for
    outputs whose values can be small next to the 2e-2 absolute bound."""
    got = from_bf16(got_bits).astype(np.float64).reshape(-1)
    ref = np.asarray(ref32, dtype=np.float64).reshape(-1)
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    e = float(np.max(np.abs(got - ref))) / scale
    assert e <= rel, f"{what}: norm-wise relative error {e:.3g} > {rel} (max |ref| {scale:.3g})"
    return e


def check_f32(got, ref, what="", rel=F32_REL):
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    assert got.shape == ref.shape
    assert np.all(np.isfinite(got) == np.isfinite(ref)), f"{what}: finiteness differs"
    fin = np.isfinite(ref)
    scale = max(float(np.max(np.abs(ref[fin]))) if fin.any() else 0.0, 1e-30)
    e = float(np.max(np.abs(got[fin] - ref[fin]))) / scale if fin.any() else 0.0
    assert e <= rel, f"{what}: norm-wise relative error {e:.3g} > {rel}"
    return e


def check_f32_elementwise(got, ref, what="", rel=F32_REL, floor=1e-30):
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    err = np.abs(got - ref)
    bad = err > rel * np.abs(ref) + floor
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond {rel} relative"


@contextlib.contextmanager
def stream_workspace(dev, nbytes, stream=None):
    """Attaches a fresh ``nbytes`` device buffer (NaN-poisoned, so a path that
    reads scratch it did not write shows up) as the stream's operator
    workspace for the duration of the block; the null stream by default."""
    import teenygrad_amd as tg
    from teenygrad_amd._lib import check, lib
    from teenygrad_amd.runtime import NULL_STREAM

    st = NULL_STREAM if stream is None else stream
    buf = dev.buffer(tg.i8, (max(int(nbytes), 256),))
    check(lib.teeny_hip_memset(buf.ptr, 0xFF, buf.nbytes, st.handle))
    st.set_workspace(buf)
    try:
        yield buf
    finally:
        st.set_workspace(None)
        st.synchronize()
        buf.free()
