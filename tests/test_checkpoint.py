"""Compressed-tensors int8 checkpoints without a GPU: the native safetensors
reader (teeny_checkpoint_*) against the independent `safetensors` package and
teeny-quant's file convention (utilities/teeny-quant/src/format.rs:16-35,
:118-126, :145-289), with the oracle as the quantizer; malformed files are
rejected with an error, never read out of bounds."""
import json
import struct

import numpy as np
import pytest

from teenygrad_amd import _lib
from teenygrad_amd.checkpoint import Checkpoint, build_config, serialize_safetensors
from teenygrad_amd._lib import TeenyError

safetensors_numpy = pytest.importorskip("safetensors.numpy")


def oracle_ct_file(orc, tensors, granularity="channel", axis=0, group_size=1, symmetric=True):
    """A teeny-quant style file, quantized by the oracle (format.rs:145-246)."""
    out, ignore = {}, []
    for name, arr in tensors.items():
        if arr.ndim < 2:
            out[name] = ("F32", arr.shape, arr.astype("<f4").tobytes())
            ignore.append(name)
            continue
        q, s, z, _ = orc.quantize_affine(arr, list(arr.shape), granularity, axis, group_size, symmetric, 8)
        out[name] = ("I8", arr.shape, q.tobytes())
        out[name + "_scale"] = ("F32", (s.size,), s.astype("<f4").tobytes())
        if not symmetric:
            out[name + "_zero_point"] = ("I32", (z.size,), z.astype("<i4").tobytes())
    cfg = build_config(granularity, axis, group_size, symmetric, sorted(ignore))
    return serialize_safetensors(out, {"quantization_config": json.dumps(cfg)}), out


def test_reader_matches_safetensors_package():
    # a file written by the `safetensors` package reads back identically
    rng = np.random.default_rng(0)
    arrays = {"a.weight": rng.standard_normal((7, 5)).astype(np.float32),
              "b": np.arange(-5, 6, dtype=np.int8), "c": rng.integers(-9, 9, (2, 3, 4)).astype(np.int32),
              "empty": np.zeros((0, 4), np.float32), "h": rng.standard_normal(6).astype(np.float16)}
    blob = safetensors_numpy.save(arrays, metadata={"k": "v", "quantization_config": json.dumps(
        build_config("channel", 0, 1, True, []))})
    with Checkpoint(image=blob) as ck:
        t = ck.tensors()
        assert set(t) == set(arrays)
        for name, arr in arrays.items():
            assert t[name]["shape"] == arr.shape
            np.testing.assert_array_equal(ck.read(name), arr)
        sch = ck.quant_scheme()
        assert sch["strategy"] == "channel" and sch["axis"] == 0 and sch["symmetric"] and sch["num_bits"] == 8
    # and our writer's output is a valid file for the package
    ours = serialize_safetensors({n: ({np.float32: "F32", np.int8: "I8", np.int32: "I32", np.float16: "F16"}[a.dtype.type],
                                      a.shape, a.tobytes()) for n, a in arrays.items()}, {"x": "y"})
    back = safetensors_numpy.load(ours)
    for name, arr in arrays.items():
        np.testing.assert_array_equal(back[name], arr)


@pytest.mark.parametrize("gran,axis,gs,sym", [("channel", 0, 1, True), ("tensor", 0, 1, True),
                                              ("group", 1, 16, True), ("channel", 1, 1, False)])
def test_teeny_quant_file_layout(orc, gran, axis, gs, sym):
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (24, 64)).astype(np.float32)
    bias = rng.normal(0, 0.1, 24).astype(np.float32)
    blob, parts = oracle_ct_file(orc, {"fc.weight": w, "fc.bias": bias}, gran, axis, gs, sym)
    with Checkpoint(image=blob) as ck:
        sch = ck.quant_scheme()
        assert sch["quant_method"] == "compressed-tensors" and sch["format"] == "int-quantized"
        assert sch["strategy"] == gran and sch["symmetric"] == sym
        t = ck.tensors()
        assert t["fc.weight"]["dtype"] == "I8" and t["fc.weight"]["shape"] == (24, 64)
        assert t["fc.weight_scale"]["dtype"] == "F32"
        assert ("fc.weight_zero_point" in t) == (not sym)
        np.testing.assert_array_equal(ck.read("fc.weight").reshape(-1).view(np.uint8),
                                      np.frombuffer(parts["fc.weight"][2], np.uint8))
        np.testing.assert_array_equal(ck.read("fc.bias"), bias)
        import ctypes
        n, k = ctypes.c_int64(), ctypes.c_int64()
        st = _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"fc.weight", ctypes.byref(n), ctypes.byref(k))
        if gran == "tensor" or (gran == "channel" and axis == 0 and sym):
            assert st == _lib.OK and (n.value, k.value) == (24, 64)
        else:
            assert st == _lib.ERR_UNSUPPORTED, _lib.last_error()
        # the bias is listed as unquantized: never a W8A16 weight
        assert _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"fc.bias", ctypes.byref(n),
                                                     ctypes.byref(k)) in (_lib.ERR_INVALID_ARGUMENT,
                                                                          _lib.ERR_UNSUPPORTED)
        assert _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"nope.weight", ctypes.byref(n),
                                                     ctypes.byref(k)) in (_lib.ERR_NOT_FOUND, _lib.ERR_UNSUPPORTED)


def header_file(header: dict, data: bytes = b"") -> bytes:
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


BAD = {
    "short": b"\x01\x02",
    "header_len_past_end": struct.pack("<Q", 1000) + b"{}",
    "header_len_zero": struct.pack("<Q", 0) + b"{}",
    "not_json": struct.pack("<Q", 4) + b"{abc",
    "not_object": header_file([1, 2]),
    "trailing": struct.pack("<Q", 4) + b"{}{}",
    "bad_dtype": header_file({"t": {"dtype": "Q8", "shape": [1], "data_offsets": [0, 1]}}, b"\0"),
    "offsets_past_data": header_file({"t": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]}}, b"\0\0"),
    "size_mismatch": header_file({"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 8),
    "negative_dim": header_file({"t": {"dtype": "I8", "shape": [-1], "data_offsets": [0, 0]}}),
    "reversed_offsets": header_file({"t": {"dtype": "I8", "shape": [0], "data_offsets": [3, 1]}}, b"\0" * 4),
    "overflow_shape": header_file({"t": {"dtype": "F32", "shape": [2 ** 40, 2 ** 40], "data_offsets": [0, 0]}}),
    "missing_offsets": header_file({"t": {"dtype": "I8", "shape": [1]}}, b"\0"),
    "metadata_not_str": header_file({"__metadata__": {"a": 1}}),
    "bad_quant_config": header_file({"__metadata__": {"quantization_config": "{not json"}}),
    "quant_config_no_groups": header_file({"__metadata__": {"quantization_config": "{\"quant_method\":\"x\"}"}}),
    "deep_nesting": struct.pack("<Q", 200) + (b"[" * 100 + b"]" * 100),
    "bad_escape": struct.pack("<Q", 9) + b'{"a\\q":1}',
    "lone_surrogate": struct.pack("<Q", 12) + b'{"\\ud800":1}',
}


@pytest.mark.parametrize("name", sorted(BAD))
def test_malformed_files_are_rejected(name):
    with pytest.raises(TeenyError) as e:
        Checkpoint(image=BAD[name])
    assert e.value.status == _lib.ERR_INVALID_ARGUMENT


def test_open_errors(tmp_path):
    import ctypes
    h = ctypes.c_void_p()
    assert _lib.lib.teeny_checkpoint_open(None, ctypes.byref(h)) == _lib.ERR_NULL_POINTER
    assert _lib.lib.teeny_checkpoint_open(str(tmp_path / "missing.safetensors").encode(),
                                          ctypes.byref(h)) == _lib.ERR_INVALID_ARGUMENT
    assert _lib.lib.teeny_checkpoint_num_tensors(None, ctypes.byref(ctypes.c_int64())) == _lib.ERR_NULL_POINTER
    assert _lib.lib.teeny_checkpoint_close(None) == _lib.OK
    # a real file on disk, read through the mapping
    p = tmp_path / "m.safetensors"
    p.write_bytes(safetensors_numpy.save({"w": np.arange(12, dtype=np.float32).reshape(3, 4)}))
    with Checkpoint(str(p)) as ck:
        np.testing.assert_array_equal(ck.read("w"), np.arange(12, dtype=np.float32).reshape(3, 4))
        assert ck.quant_scheme() is None
        with pytest.raises(KeyError):
            ck.read("v")
        idx = ctypes.c_int64()
        assert _lib.lib.teeny_checkpoint_find(ck.handle, b"v", ctypes.byref(idx)) == _lib.ERR_NOT_FOUND
        buf = np.empty(11, np.float32)
        assert _lib.lib.teeny_checkpoint_read(ck.handle, 0, buf.ctypes.data, 44, 0, None) == _lib.ERR_SHAPE_MISMATCH
        assert _lib.lib.teeny_checkpoint_read(ck.handle, 5, buf.ctypes.data, 44, 0, None) == _lib.ERR_INVALID_ARGUMENT


def _scheme_file(weights: dict, extra=None) -> bytes:
    """A file with fc.weight I8 [4, 8] + fc.weight_scale F32 [4] under a
    quantization_config whose weights block is `weights`."""
    t = {"fc.weight": ("I8", (4, 8), bytes(32)), "fc.weight_scale": ("F32", (4,), bytes(16))}
    t.update(extra or {})
    cfg = {"quant_method": "compressed-tensors", "format": "int-quantized",
           "config_groups": {"group_0": {"weights": weights, "targets": ["*"]}}}
    return serialize_safetensors(t, {"quantization_config": json.dumps(cfg)})


@pytest.mark.parametrize("sym", [None, "yes", 1])
def test_scheme_without_bool_symmetric_is_rejected(sym):
    # WeightsConfig.symmetric is a required bool (format.rs:52-70): a file
    # that does not state it does not say whether zero points exist
    w = {"num_bits": 8, "type": "int", "strategy": "channel", "axis": 0}
    if sym is not None:
        w["symmetric"] = sym
    with pytest.raises(TeenyError) as e:
        Checkpoint(image=_scheme_file(w))
    assert e.value.status == _lib.ERR_INVALID_ARGUMENT
    assert "symmetric" in str(e.value)


@pytest.mark.parametrize("strategy", ["channel", "group"])
def test_strategy_without_axis_is_ambiguous(strategy):
    # granularity_from_config rejects channel / group without an axis
    # (validate.rs:94-103); neither the W8A16 loader nor dequantize guesses 0
    import ctypes
    w = {"num_bits": 8, "type": "int", "symmetric": True, "strategy": strategy}
    if strategy == "group":
        w["group_size"] = 4
    with Checkpoint(image=_scheme_file(w)) as ck:
        assert ck.quant_scheme()["axis"] == -1
        n, k = ctypes.c_int64(), ctypes.c_int64()
        assert _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"fc.weight", ctypes.byref(n),
                                                     ctypes.byref(k)) == _lib.ERR_INVALID_ARGUMENT
        assert "axis" in _lib.last_error()
        with pytest.raises(ValueError, match="axis"):
            ck.dequantize("fc.weight")


def test_zero_point_under_symmetric_scheme_is_rejected():
    # a symmetric scheme omits the zero points (format.rs:25-26): a file that
    # carries them anyway is inconsistent and not loaded as W8A16
    import ctypes
    w = {"num_bits": 8, "type": "int", "symmetric": True, "strategy": "channel", "axis": 0}
    blob = _scheme_file(w, {"fc.weight_zero_point": ("I32", (4,), bytes(16))})
    with Checkpoint(image=blob) as ck:
        n, k = ctypes.c_int64(), ctypes.c_int64()
        assert _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"fc.weight", ctypes.byref(n),
                                                     ctypes.byref(k)) == _lib.ERR_INVALID_ARGUMENT
        assert "zero_point" in _lib.last_error()
    # the same file without it loads
    with Checkpoint(image=_scheme_file(w)) as ck:
        n, k = ctypes.c_int64(), ctypes.c_int64()
        assert _lib.lib.teeny_checkpoint_w8a16_shape(ck.handle, b"fc.weight", ctypes.byref(n),
                                                     ctypes.byref(k)) == _lib.OK
        assert (n.value, k.value) == (4, 8)
