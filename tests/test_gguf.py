"""GGUF files: the library's parser (host only, no GPU) against files written
by tests/gguf_writer.py, its refusals of malformed input, and the typed
oracle decode against the same model with its weights decoded to fp32."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2

CFG = dict(layers=2, dim=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=96, max_seq=32,
           rope_base=10000.0, eps=1e-5)
TYPES = dict(tok_embed=gw.Q4_K, wq=gw.Q4_K, wk=gw.Q4_K, wv=gw.Q6_K, wo=gw.Q4_K, w_gate=gw.Q4_K, w_up=gw.Q4_K,
             w_down=gw.Q6_K, lm_head=gw.Q6_K)


@pytest.fixture(scope="module")
def lib():
    from aljabr_amd import abi
    return abi.load()


def _open(lib, path):
    h = ctypes.c_void_p()
    rc = lib.aljabr_rocm_gguf_open(path.encode(), ctypes.byref(h))
    return rc, h


def test_parse_written_model(lib, oracle, tmp_path):
    meta, tensors, _ = gw.llama_model(oracle, CFG, TYPES)
    path = str(tmp_path / "m.gguf")
    gw.write_gguf(path, meta, tensors)
    rc, h = _open(lib, path)
    assert rc == 0
    try:
        n = ctypes.c_int64()
        assert lib.aljabr_rocm_gguf_tensor_count(h, ctypes.byref(n)) == 0 and n.value == len(tensors)
        v = ctypes.c_int64()
        assert lib.aljabr_rocm_gguf_meta_int(h, b"llama.block_count", ctypes.byref(v)) == 0 and v.value == 2
        assert lib.aljabr_rocm_gguf_meta_int(h, b"tokenizer.ggml.tokens", ctypes.byref(v)) == 0 and v.value == 8
        f = ctypes.c_double()
        assert lib.aljabr_rocm_gguf_meta_float(h, b"llama.rope.freq_base", ctypes.byref(f)) == 0
        assert f.value == 10000.0
        buf = ctypes.create_string_buffer(32)
        assert lib.aljabr_rocm_gguf_meta_string(h, b"general.architecture", buf, 32) == 0 and buf.value == b"llama"
        with open(path, "rb") as fh:
            raw = fh.read()
        for i, (name, dims, gtype, data) in enumerate(tensors):
            idx = ctypes.c_int64()
            assert lib.aljabr_rocm_gguf_find_tensor(h, name.encode(), ctypes.byref(idx)) == 0 and idx.value == i
            nm = ctypes.create_string_buffer(96)
            t, nd = ctypes.c_int32(), ctypes.c_int32()
            d = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            assert lib.aljabr_rocm_gguf_tensor_info(h, i, nm, 96, ctypes.byref(t), ctypes.byref(nd), d,
                                                    ctypes.byref(off), ctypes.byref(nb)) == 0
            assert nm.value.decode() == name and t.value == gtype and nd.value == len(dims)
            assert list(d)[:len(dims)] == dims and nb.value == len(data)
            assert raw[off.value:off.value + nb.value] == data
            assert off.value % gw.ALIGN == 0
    finally:
        lib.aljabr_rocm_gguf_close(h)


@pytest.mark.parametrize("damage", ["magic", "version", "truncated_meta", "truncated_table", "data_past_end",
                                    "unknown_type", "empty"])
def test_parser_refuses_malformed(lib, oracle, tmp_path, damage):
    meta, tensors, _ = gw.llama_model(oracle, dict(CFG, layers=1), TYPES)
    path = str(tmp_path / "m.gguf")
    gw.write_gguf(path, meta, tensors)
    raw = bytearray(open(path, "rb").read())
    if damage == "magic":
        raw[0:4] = b"GGUX"
    elif damage == "version":
        raw[4:8] = (7).to_bytes(4, "little")
    elif damage == "truncated_meta":
        raw = raw[:60]
    elif damage == "truncated_table":
        raw = raw[:900]
    elif damage == "data_past_end":
        raw = raw[:len(raw) - 4096]
    elif damage == "unknown_type":
        gw.write_gguf(path, meta, [(tensors[0][0], tensors[0][1], 99, tensors[0][3])])
        raw = bytearray(open(path, "rb").read())
    else:
        raw = bytearray()
    with open(path, "wb") as f:
        f.write(bytes(raw))
    rc, h = _open(lib, path)
    assert rc in (-2, -3) and not h.value
    assert rc == (-3 if damage == "unknown_type" else -2)


def test_missing_file(lib, tmp_path):
    rc, h = _open(lib, str(tmp_path / "absent.gguf"))
    assert rc == -2 and not h.value


def test_typed_oracle_matches_dequantized_weights(oracle):
    """The typed step with Q4_K/Q6_K/Q8_0 tensors equals the same model with
    every tensor decoded to fp32 first (pins the per-type dispatch of the
    matvecs and of the embedding row)."""
    types = dict(TYPES, wk=gw.Q8_0, wo=gw.Q4_0, tok_embed=gw.Q6_K)
    cfg = dict(CFG)
    _, _, w = gw.llama_model(oracle, cfg, types, seed=3)
    shapes = {"wq": (256, 256), "wk": (128, 256), "wv": (128, 256), "wo": (256, 256), "w_gate": (512, 256),
              "w_up": (512, 256), "w_down": (256, 512)}

    def to_f32(pair, n, k):
        t, arr = pair
        if t == gw.F32:
            return pair
        if t == gw.F16:
            return (gw.F32, arr.view(np.float16).astype(np.float32))
        return (gw.F32, oracle.dequant(t, arr, n * k))

    w32 = dict(w)
    for key, (n, k) in shapes.items():
        w32[key] = [to_f32(p, n, k) for p in w[key]]
    w32["tok_embed"] = to_f32(w["tok_embed"], cfg["vocab"], cfg["dim"])
    w32["lm_head"] = to_f32(w["lm_head"], cfg["vocab"], cfg["dim"])
    a, b = oracle.TypedLlamaOracle(cfg, w), oracle.TypedLlamaOracle(cfg, w32)
    tok = 5
    for pos in range(4):
        ta, la, _ = a.decode(tok, pos)
        tb, lb, _ = b.decode(tok, pos)
        assert np.isfinite(la).all()
        assert rel_l2(la, lb) < 1e-5 and ta == tb
        tok = ta
