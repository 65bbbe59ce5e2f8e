"""Pins the oracle's teeny-quant restatement (bit-exact int8 / intN).

The reference ships no int8 golden vectors.  The oracle is pinned by
(1) hand-derived known answers (tests/quant_cases.py), (2) a second,
independently written numpy restatement on random data with planted ties,
(3) the reference's own unit-test invariants and error cases
(utilities/teeny-quant/src/quant/affine.rs:163-288,
utilities/teeny-quant/tests/quantize_roundtrip.rs:32-174).
"""
import numpy as np
import pytest

from quant_cases import KNOWN, group_ids, numpy_quantize

ERR_SHAPE_MISMATCH, ERR_INVALID_AXIS, ERR_INVALID_GROUP_SIZE = 4, 6, 7


@pytest.mark.parametrize("case", KNOWN, ids=[c[0] for c in KNOWN])
def test_known_answers(orc, case):
    name, data, shape, gran, axis, gs, sym, bits, want_q, want_s, want_z = case
    q, s, z, g = orc.quantize_affine(np.array(data, np.float32), shape, gran, axis, gs, sym, bits)
    np.testing.assert_array_equal(q, np.array(want_q, np.int8))
    np.testing.assert_array_equal(s, np.array(want_s, np.float32))
    np.testing.assert_array_equal(z, np.array(want_z, np.int32))
    np.testing.assert_array_equal(g, group_ids(shape, gran, axis, gs)[0].astype(np.uint32))


RANDOM_CASES = [
    ((64, 96), "channel", 0, 1, True, 8),
    ((64, 96), "channel", 1, 1, True, 8),
    ((64, 96), "tensor", 0, 1, False, 8),
    ((8, 5, 33), "group", 2, 8, True, 8),
    ((8, 5, 33), "group", 1, 2, False, 4),
    ((8, 5, 33), "group", 0, 3, True, 4),
    ((256, 256, 3, 3), "channel", 0, 1, True, 8),
]


@pytest.mark.parametrize("shape,gran,axis,gs,sym,bits", RANDOM_CASES)
def test_matches_numpy_restatement(orc, shape, gran, axis, gs, sym, bits):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 0.02, shape).astype(np.float32)
    # plant exact ties: scale the first element of every group to the group's amax
    # and put x = +-k.5 * scale values in
    x.reshape(-1)[::7] *= 3.0
    q, s, z, g = orc.quantize_affine(x, shape, gran, axis, gs, sym, bits)
    nq, ns, nz, ng = numpy_quantize(x, shape, gran, axis, gs, sym, bits)
    np.testing.assert_array_equal(g, ng)
    np.testing.assert_array_equal(s, ns)
    np.testing.assert_array_equal(z, nz)
    np.testing.assert_array_equal(q, nq)


def test_planted_ties_round_half_away(orc):
    # scale 1 per channel (amax 127): every .5 must round away from zero
    halves = np.arange(-126.5, 127.0, 1.0, dtype=np.float32)
    x = np.stack([np.concatenate([[127.0], halves[:200]]), np.concatenate([[-127.0], halves[-200:]])])
    q, s, _, _ = orc.quantize_affine(x, x.shape, "channel", 0)
    np.testing.assert_array_equal(s, [1.0, 1.0])
    want = np.trunc(x) + np.sign(x) * (np.abs(x - np.trunc(x)) >= 0.5)
    np.testing.assert_array_equal(q, np.clip(want, -127, 127).astype(np.int8).reshape(-1))


def test_dequantize_exact(orc):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (6, 10)).astype(np.float32)
    for sym in (True, False):
        q, s, z, _ = orc.quantize_affine(x, x.shape, "channel", 0, symmetric=sym)
        deq = orc.dequantize_affine(q, s, z, x.shape, "channel", 0)
        want = (q.reshape(6, 10).astype(np.int32) - z[:, None]).astype(np.float32) * s[:, None]
        np.testing.assert_array_equal(deq, want)


# ── the reference's unit tests (affine.rs:163-288) ──────────────────────────


def test_ref_per_tensor_symmetric_round_trip(orc):
    data = np.array([-1.0, -0.5, 0.0, 0.5, 1.0, 2.0], np.float32)
    q, s, z, _ = orc.quantize_affine(data, [6], "tensor", symmetric=True)
    assert s.size == 1 and z[0] == 0
    back = orc.dequantize_affine(q, s, z, [6], "tensor")
    assert np.all(np.abs(data - back) < 0.02)


def test_ref_per_tensor_asymmetric_positive_range(orc):
    data = np.array([0.0, 1.0, 2.0, 3.0, 4.0], np.float32)
    q, s, z, _ = orc.quantize_affine(data, [5], "tensor", symmetric=False)
    back = orc.dequantize_affine(q, s, z, [5], "tensor")
    assert np.all(np.abs(data - back) < 0.05)


def test_ref_per_channel_independent_scales(orc):
    data = np.array([0.1, -0.1, 0.05, -0.05, 100.0, -100.0, 50.0, -50.0], np.float32)
    q, s, z, _ = orc.quantize_affine(data, [2, 4], "channel", 0)
    assert s.size == 2
    back = orc.dequantize_affine(q, s, z, [2, 4], "channel", 0).reshape(-1)
    assert np.all(np.abs(data - back) < np.maximum(np.abs(data), 1.0) * 0.02)


def test_ref_group_matches_per_channel(orc):
    data = np.arange(8, dtype=np.float32) - 4.0
    a = orc.quantize_affine(data, [2, 4], "channel", 0)
    b = orc.quantize_affine(data, [2, 4], "group", 1, group_size=4)
    assert a[1].size == b[1].size == 2
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_ref_errors(orc):
    data = np.ones(4, np.float32)
    with pytest.raises(orc.OracleError) as e:
        orc.quantize_affine(data, [4], "group", 0, group_size=0)
    assert e.value.status == ERR_INVALID_GROUP_SIZE
    with pytest.raises(orc.OracleError) as e:
        orc.quantize_affine(data, [4], "channel", 3)
    assert e.value.status == ERR_INVALID_AXIS


def test_ref_int4_clamped(orc):
    q, _, _, _ = orc.quantize_affine(np.array([-100.0, 100.0], np.float32), [2], "tensor", bits=4)
    assert np.all((q >= -7) & (q <= 7))


@pytest.mark.parametrize("gran,axis,gs,sym,bits,tol", [
    ("channel", 0, 1, True, 8, 0.05),   # quantize_roundtrip.rs:145-152
    ("tensor", 0, 1, False, 8, 0.05),   # :155-161
    ("group", 1, 4, True, 4, 0.5),      # :164-173
])
def test_ref_checkpoint_round_trip(orc, gran, axis, gs, sym, bits, tol):
    # the 4 x 8 weight of quantize_roundtrip.rs:32-36: (i - 16) * 0.37
    w = ((np.arange(32, dtype=np.float32) - 16.0) * np.float32(0.37)).reshape(4, 8)
    q, s, z, _ = orc.quantize_affine(w, [4, 8], gran, axis, gs, sym, bits)
    back = orc.dequantize_affine(q, s, z, [4, 8], gran, axis, gs)
    assert np.all(np.abs(w - back) <= np.maximum(np.abs(w), 1.0) * tol)


def test_quant_sensitivity(orc):
    # half-to-even rounding or a dropped zero point must disagree with the oracle
    x = np.array([127.0, 2.5, 0.5, -1.5], np.float32)
    q, _, _, _ = orc.quantize_affine(x, [4], "tensor")
    assert not np.array_equal(q, np.round(x).astype(np.int8))
    xa = np.array([-100.0, 155.0, 20.5], np.float32)
    qa, sa, za, _ = orc.quantize_affine(xa, [3], "tensor", symmetric=False)
    assert za[0] != 0 and not np.array_equal(qa, np.clip(np.round(xa / sa[0]), -128, 127).astype(np.int8))
