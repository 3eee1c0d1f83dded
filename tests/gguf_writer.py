"""GGUF v3 writer and synthetic Llama-family model files for the tests.

TEST INFRASTRUCTURE. Writes the layout the reference's parser reads
(engine/gguf/aljabr-gguf-core/.../loader/GGUFParser.java:18-63 and the
GGUFWriter that produces it, engine/gguf/aljabr-gguf-core/.../writer/
GGUFWriter.java): "GGUF", u32 version 3, u64 tensor count, u64 KV count, KV
pairs (u64-length string key, u32 value type, value), tensor infos (name,
u32 n_dims, u64 dims with dims[0] the row length, u32 ggml type, u64 offset
from the data start), zero padding to general.alignment (32), tensor data at
aligned offsets. All little endian.
"""
from __future__ import annotations

import struct

import numpy as np

ALIGN = 32
# GGUF value types.
U32, I32, F32V, BOOL, STRING, ARRAY, U64 = 4, 5, 6, 7, 8, 9, 10
# ggml tensor types (= ALJABR_ROCM_TYPE_* ids).
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == U32:
        return struct.pack("<I", value)
    if vtype == I32:
        return struct.pack("<i", value)
    if vtype == F32V:
        return struct.pack("<f", value)
    if vtype == BOOL:
        return struct.pack("<B", 1 if value else 0)
    if vtype == STRING:
        return _str(value)
    if vtype == U64:
        return struct.pack("<Q", value)
    if vtype == ARRAY:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, v) for v in items)
    raise ValueError(f"value type {vtype}")


def write_gguf(path: str, meta: list, tensors: list, version: int = 3) -> None:
    """meta: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, raw bytes)]
    with dims in GGUF order (dims[0] = row length)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, vtype, value in meta:
        out += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offset = 0
    offsets = []
    for name, dims, gtype, data in tensors:
        offsets.append(offset)
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gtype, offset)
        offset += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    out += b"\0" * ((-len(out)) % ALIGN)
    for (name, dims, gtype, data), off in zip(tensors, offsets):
        assert len(out) % ALIGN == 0
        out += data
        out += b"\0" * ((-len(out)) % ALIGN)
    with open(path, "wb") as f:
        f.write(bytes(out))


def _matrix(oracle, gtype: int, n: int, k: int, seed: int, std: float) -> np.ndarray:
    """Raw [n][k] matrix of a ggml type: quantized blocks (uint8) or values."""
    if gtype in (Q4_K, Q6_K):
        # Random codes: Q4_K weights have rms ~300 d, Q6_K ~1400 d.
        return oracle.random_k_blocks(gtype, n * k // 256, seed, scale=std / (200 if gtype == Q4_K else 1000))
    w = oracle.normal(seed, n * k, 0.0, std)
    if gtype in (Q4_0, Q8_0):
        return oracle.quantize(gtype, w)
    if gtype == F16:
        return w.astype(np.float16).view(np.uint16)
    return w


def llama_model(oracle, cfg: dict, types: dict, seed: int = 1):
    """A synthetic Llama-family model: returns (meta, tensors, weights) where
    meta/tensors feed write_gguf and weights feed oracle.TypedLlamaOracle.
    `types` maps tok_embed, lm_head (None: tied to tok_embed) and the matrix
    names wq, wk, wv, wo, w_gate, w_up, w_down to ggml types."""
    dim, ffn, nh, nkv, hd, vocab, L = (cfg[k] for k in ("dim", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab",
                                                         "layers"))
    qd, kvd = nh * hd, nkv * hd
    meta = [("general.architecture", STRING, "llama"),
            ("general.alignment", U32, ALIGN),
            ("llama.block_count", U32, L),
            ("llama.context_length", U32, cfg["max_seq"]),
            ("llama.embedding_length", U32, dim),
            ("llama.feed_forward_length", U32, ffn),
            ("llama.attention.head_count", U32, nh),
            ("llama.attention.head_count_kv", U32, nkv),
            ("llama.rope.freq_base", F32V, cfg["rope_base"]),
            ("llama.attention.layer_norm_rms_epsilon", F32V, cfg["eps"]),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(8)]))]
    if hd != dim // nh:
        meta.append(("llama.attention.key_length", U32, hd))
    tensors, weights = [], {k: [] for k in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up",
                                            "w_down")}
    s = seed * 1000
    key_index = {k: i for i, k in enumerate(("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"))}

    def add(name, dims, gtype, arr):
        tensors.append((name, dims, gtype, np.ascontiguousarray(arr).tobytes()))

    emb_t = types["tok_embed"]
    emb = _matrix(oracle, emb_t, vocab, dim, s, 1.0)
    add("token_embd.weight", [dim, vocab], emb_t, emb)
    weights["tok_embed"] = (emb_t, emb)
    shapes = {"wq": (qd, dim, "attn_q"), "wk": (kvd, dim, "attn_k"), "wv": (kvd, dim, "attn_v"),
              "wo": (dim, qd, "attn_output"), "w_gate": (ffn, dim, "ffn_gate"), "w_up": (ffn, dim, "ffn_up"),
              "w_down": (dim, ffn, "ffn_down")}
    for l in range(L):
        an = (1.0 + 0.1 * oracle.normal(s + 10 * l + 1, dim)).astype(np.float32)
        fn = (1.0 + 0.1 * oracle.normal(s + 10 * l + 2, dim)).astype(np.float32)
        add(f"blk.{l}.attn_norm.weight", [dim], F32, an)
        weights["attn_norm"].append(an)
        for key in ("wq", "wk", "wv", "wo"):
            n, k, gname = shapes[key]
            t = types[key]
            m = _matrix(oracle, t, n, k, s + 100 * l + 11 * key_index[key], 0.5 / np.sqrt(k))
            add(f"blk.{l}.{gname}.weight", [k, n], t, m)
            weights[key].append((t, m))
        add(f"blk.{l}.ffn_norm.weight", [dim], F32, fn)
        weights["ffn_norm"].append(fn)
        for key in ("w_gate", "w_up", "w_down"):
            n, k, gname = shapes[key]
            t = types[key]
            m = _matrix(oracle, t, n, k, s + 100 * l + 11 * key_index[key], 0.5 / np.sqrt(k))
            add(f"blk.{l}.{gname}.weight", [k, n], t, m)
            weights[key].append((t, m))
    on = (1.0 + 0.1 * oracle.normal(s + 7, dim)).astype(np.float32)
    add("output_norm.weight", [dim], F32, on)
    weights["out_norm"] = on
    lm_t = types.get("lm_head")
    if lm_t is None:
        weights["lm_head"] = weights["tok_embed"]
    else:
        lm = _matrix(oracle, lm_t, vocab, dim, s + 9, 0.5 / np.sqrt(dim))
        add("output.weight", [dim, vocab], lm_t, lm)
        weights["lm_head"] = (lm_t, lm)
    return meta, tensors, weights
