"""The safetensors reader behind aljabr_rocm_safetensors_* (host code, no GPU):
files written by the `safetensors` library itself and by the test writer
parse to the same names, dtypes, shapes and bytes; metadata reads back; and
malformed files (SafetensorHeaderParser / SafetensorValidator's checks:
header length, offsets against shape and dtype, overlaps, unknown dtypes,
non-integer shapes, trailing bytes) are rejected with -2."""
from __future__ import annotations

import ctypes
import json
import struct

import numpy as np
import pytest

import safetensors_writer as sw
from aljabr_amd import abi


class _File:
    def __init__(self, path):
        self.lib = abi.load()
        self.h = ctypes.c_void_p()
        abi.check(self.lib.aljabr_rocm_safetensors_open(path.encode(), ctypes.byref(self.h)), "open")

    def close(self):
        self.lib.aljabr_rocm_safetensors_close(self.h)

    def tensors(self):
        n = ctypes.c_int64()
        abi.check(self.lib.aljabr_rocm_safetensors_tensor_count(self.h, ctypes.byref(n)), "count")
        out = {}
        for i in range(n.value):
            name = ctypes.create_string_buffer(256)
            dt, nd = ctypes.c_int32(), ctypes.c_int32()
            dims = (ctypes.c_int64 * 8)()
            nbytes = ctypes.c_uint64()
            abi.check(self.lib.aljabr_rocm_safetensors_tensor_info(self.h, i, name, 256, ctypes.byref(dt),
                                                                   ctypes.byref(nd), dims, ctypes.byref(nbytes)), "info")
            ptr = ctypes.c_void_p()
            abi.check(self.lib.aljabr_rocm_safetensors_tensor_data(self.h, i, ctypes.byref(ptr)), "data")
            raw = ctypes.string_at(ptr.value, nbytes.value) if nbytes.value else b""
            out[name.value.decode()] = (sw.DTYPES[dt.value], list(dims[:nd.value]), raw)
        return out


def _status(path):
    h = ctypes.c_void_p()
    return abi.load().aljabr_rocm_safetensors_open(path.encode(), ctypes.byref(h))


def test_files_from_the_safetensors_library(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(1)
    arrays = {"model.embed_tokens.weight": rng.standard_normal((16, 8)).astype(np.float32),
              "a.half": rng.standard_normal((3, 5, 2)).astype(np.float16),
              "codes.qweight": rng.integers(0, 256, (4, 64), dtype=np.uint8),
              "ids": np.arange(7, dtype=np.int64), "scalar": np.array(3.5, np.float64),
              "empty": np.zeros((0, 4), np.float32)}
    path = str(tmp_path / "lib.safetensors")
    save_file(arrays, path, metadata={"format": "pt", "note": "café"})
    f = _File(path)
    got = f.tensors()
    names = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.uint8): "U8",
             np.dtype(np.int64): "I64", np.dtype(np.float64): "F64"}
    assert set(got) == set(arrays)
    for k, a in arrays.items():
        dt, shape, raw = got[k]
        assert dt == names[a.dtype] and shape == list(a.shape) and raw == a.tobytes(), k
    buf = ctypes.create_string_buffer(64)
    abi.check(f.lib.aljabr_rocm_safetensors_meta(f.h, b"note", buf, 64), "meta")
    assert buf.value.decode() == "café"
    idx = ctypes.c_int64()
    abi.check(f.lib.aljabr_rocm_safetensors_find_tensor(f.h, b"ids", ctypes.byref(idx)), "find")
    assert got["ids"][2] == np.arange(7, dtype=np.int64).tobytes()
    assert f.lib.aljabr_rocm_safetensors_find_tensor(f.h, b"nope", ctypes.byref(idx)) == abi.ERR_BAD_ARGUMENT
    f.close()


def test_writer_round_trip_with_bf16(tmp_path):
    x = np.linspace(-3, 3, 24, dtype=np.float32)
    bits = sw.bf16_bits(x)
    assert np.abs(sw.bf16_to_f32(bits) - x).max() <= 2 ** -8 * 3
    path = str(tmp_path / "w.safetensors")
    sw.write(path, [("x", "BF16", (4, 6), bits.tobytes()), ("flag", "BOOL", (2,), b"\x01\x00")], {"k": "v"})
    got = _File(path).tensors()
    assert got["x"] == ("BF16", [4, 6], bits.tobytes())
    assert got["flag"] == ("BOOL", [2], b"\x01\x00")


def _raw(path, header: dict, data: bytes, pad=b""):
    text = json.dumps(header).encode() + pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + data)


@pytest.mark.parametrize("case", ["short_data", "size_mismatch", "overlap", "dtype", "float_shape", "negative_dim",
                                  "trailing", "not_object", "header_too_long", "missing_offsets", "bad_escape",
                                  "duplicate"])
def test_malformed_files_are_rejected(tmp_path, case):
    path = str(tmp_path / f"{case}.safetensors")
    ok = {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}
    data = bytes(32)
    if case == "short_data":
        _raw(path, {"t": {"dtype": "F32", "shape": [4, 4], "data_offsets": [0, 64]}}, data)
    elif case == "size_mismatch":
        _raw(path, {"t": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 16]}}, data)
    elif case == "overlap":
        _raw(path, {"a": ok, "b": {"dtype": "F32", "shape": [2, 2], "data_offsets": [8, 24]}}, data)
    elif case == "dtype":
        _raw(path, {"t": {"dtype": "F17", "shape": [2, 2], "data_offsets": [0, 16]}}, data)
    elif case == "float_shape":
        with open(path, "wb") as f:
            text = b'{"t": {"dtype": "F32", "shape": [2.0, 2], "data_offsets": [0, 16]}}'
            f.write(struct.pack("<Q", len(text)) + text + data)
    elif case == "negative_dim":
        _raw(path, {"t": {"dtype": "F32", "shape": [-2, -2], "data_offsets": [0, 16]}}, data)
    elif case == "trailing":
        _raw(path, {"t": ok}, data, pad=b" x")
    elif case == "not_object":
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", 2) + b"[]" + data)
    elif case == "header_too_long":
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", 1 << 40) + b"{}" + data)
    elif case == "missing_offsets":
        _raw(path, {"t": {"dtype": "F32", "shape": [2, 2]}}, data)
    elif case == "duplicate":
        with open(path, "wb") as f:
            e = b'{"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}'
            e2 = b'{"dtype": "F32", "shape": [2, 2], "data_offsets": [16, 32]}'
            text = b'{"t": ' + e + b', "t": ' + e2 + b'}'
            f.write(struct.pack("<Q", len(text)) + text + data)
    elif case == "bad_escape":
        with open(path, "wb") as f:
            text = b'{"t\\q": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]}}'
            f.write(struct.pack("<Q", len(text)) + text + data)
    assert _status(path) == abi.ERR_BAD_ARGUMENT
    assert abi.last_error()


def test_missing_file(tmp_path):
    assert _status(str(tmp_path / "absent.safetensors")) == abi.ERR_BAD_ARGUMENT
