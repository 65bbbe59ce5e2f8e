"""Known-answer cases for teeny-quant affine quantization.

Each expected value is derived by hand from the reference's formulas
(utilities/teeny-quant/src/quant/affine.rs:47-161) on inputs chosen so that
every division is exact in fp32 (scale 1) or resolves to an exact tie —
which is where a half-to-even rounding, a missing zero-point, a wrong
clamp range or a NaN/inf slip would show — plus the round-trip and error
cases of the reference's own unit tests (affine.rs:163-288,
tests/quantize_roundtrip.rs:32-174).
"""
import numpy as np

# name, data, shape, granularity, axis, group_size, symmetric, bits, q, scales, zero_points
KNOWN = [
    # amax = 127 -> scale = 1: q = round_half_away(x); ties go away from zero
    # (0.49999997 is the largest fp32 below 0.5: floor(x + 0.5) would wrongly give 1)
    ("ties_half_away", [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 62.5, 0.49999997], [8], "tensor", 0, 1,
     True, 8, [127, 3, -3, 1, -1, 2, 63, 0], [1.0], [0]),
    # asymmetric, lo = -100, hi = 155: scale = 255/255 = 1, zp = round(-128 + 100) = -28
    ("asym_exact", [-100.0, 155.0, 0.5, -0.5, 20.5], [5], "tensor", 0, 1, False, 8,
     [-128, 127, -27, -29, -7], [1.0], [-28]),
    # affine.rs:167-178 data: amax = 2, scale = f32(2/127); -1/scale is exactly -63.5 in fp32
    ("ref_unit_per_tensor", [-1.0, -0.5, 0.0, 0.5, 1.0, 2.0], [6], "tensor", 0, 1, True, 8,
     [-64, -32, 0, 32, 64, 127], [np.float32(2.0) / np.float32(127.0)], [0]),
    # NaN is skipped by min/max and quantizes to 0 (Rust `NaN as i32` == 0)
    ("nan", [float("nan"), 1.0, -2.0], [3], "tensor", 0, 1, True, 8, [0, 64, -127],
     [np.float32(2.0) / np.float32(127.0)], [0]),
    # +inf: scale = inf, x/scale is NaN (inf/inf) or 0 -> q = 0
    ("inf", [float("inf"), 1.0], [2], "tensor", 0, 1, True, 8, [0, 0], [float("inf")], [0]),
    # all-zero group: amax == 0 -> scale 1
    ("zeros", [0.0, 0.0, 0.0, 0.0], [2, 2], "channel", 0, 1, True, 8, [0, 0, 0, 0], [1.0, 1.0], [0, 0]),
    # per-channel over axis 1 of [2, 3]: group = column
    ("per_channel_axis1", [1.0, -2.0, 3.0, -1.0, 2.0, -3.0], [2, 3], "channel", 1, 1, True, 8,
     [127, -127, 127, -127, 127, -127],
     [np.float32(1.0) / np.float32(127.0), np.float32(2.0) / np.float32(127.0),
      np.float32(3.0) / np.float32(127.0)], [0, 0, 0]),
    # group-wise along axis 1, group_size 2, shape [2, 3]: groups per row ceil(3/2) = 2;
    # row 0 -> groups 0 (cols 0,1) and 1 (col 2); row 1 -> 2 and 3
    ("group_ragged", [127.0, 63.5, 10.0, -127.0, 0.5, -10.0], [2, 3], "group", 1, 2, True, 8,
     [127, 64, 127, -127, 1, -127], [1.0, np.float32(10.0) / np.float32(127.0), 1.0,
                                     np.float32(10.0) / np.float32(127.0)], [0, 0, 0, 0]),
    # int4 (affine.rs:279-287): amax 100 -> scale 100/7, q = +-7 within [-7, 7]
    ("int4_clamp", [-100.0, 100.0], [2], "tensor", 0, 1, True, 4, [-7, 7],
     [np.float32(100.0) / np.float32(7.0)], [0]),
    # asymmetric int4: lo = -8, hi = 7 -> scale = 15/15 = 1, zp = round(-8 + 8) = 0
    ("int4_asym", [-8.0, 7.0, 0.5, -3.5], [4], "tensor", 0, 1, False, 4, [-8, 7, 1, -4], [1.0], [0]),
]


def group_ids(shape, granularity, axis, group_size):
    """Independent numpy statement of groups.rs:78-100."""
    idx = np.indices(shape).reshape(len(shape), -1)
    if granularity == "tensor":
        return np.zeros(idx.shape[1], dtype=np.int64), 1
    if granularity == "channel":
        return idx[axis].astype(np.int64), shape[axis]
    other = [d for d in range(len(shape)) if d != axis]
    outer = np.ravel_multi_index([idx[d] for d in other], [shape[d] for d in other]) if other else np.zeros(idx.shape[1], np.int64)
    along = -(-shape[axis] // group_size)
    n_outer = int(np.prod([shape[d] for d in other])) if other else 1
    return outer * along + idx[axis] // group_size, n_outer * along


def numpy_quantize(data, shape, granularity, axis, group_size, symmetric, bits):
    """A second, vectorised restatement (fp32 numpy arithmetic; NaN-free data)."""
    x = np.asarray(data, dtype=np.float32).reshape(-1)
    g, ng = group_ids(shape, granularity, axis, group_size)
    qmax = (1 << (bits - 1)) - 1
    qmin = -qmax if symmetric else -qmax - 1
    vmin = np.full(ng, np.inf, np.float32)
    vmax = np.full(ng, -np.inf, np.float32)
    np.minimum.at(vmin, g, x)
    np.maximum.at(vmax, g, x)
    fin = np.isfinite(vmin)
    lo = np.where(fin, np.minimum(vmin, np.float32(0)), np.float32(0)).astype(np.float32)
    hi = np.where(fin, np.maximum(vmax, np.float32(0)), np.float32(0)).astype(np.float32)

    def rnd(v):
        t = np.trunc(v)
        return np.where(np.abs(v - t) >= 0.5, t + np.sign(v), t)

    if symmetric:
        amax = np.maximum(np.abs(lo), np.abs(hi))
        scale = np.where(amax == 0, np.float32(1), amax / np.float32(qmax)).astype(np.float32)
        zp = np.zeros(ng, np.int64)
    else:
        scale = np.where(hi == lo, np.float32(1), (hi - lo) / np.float32(qmax - qmin)).astype(np.float32)
        zp = np.clip(rnd(np.float32(qmin) - lo / scale).astype(np.int64), qmin, qmax)
    q = np.clip(rnd(x / scale[g]).astype(np.int64) + zp[g], qmin, qmax).astype(np.int8)
    return q, scale, zp.astype(np.int32), g.astype(np.uint32)
