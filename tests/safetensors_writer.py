"""safetensors writer for the tests (TEST INFRASTRUCTURE): the layout the
reference's parser reads (engine/safetensor/aljabr-safetensor-loader/.../
SafetensorHeaderParser.java:13-24): u64 little-endian header length, JSON
header {name: {"dtype", "shape", "data_offsets": [begin, end]}, optional
"__metadata__"}, then the tensor bytes. Writes any dtype (BF16 included) and,
for the parser's error tests, deliberately broken headers."""
from __future__ import annotations

import json
import struct

import numpy as np

# (dtype name, bytes per element) in the reference's SafetensorDType order.
DTYPES = ["BF16", "F16", "F32", "F64", "F8_E4M3", "F8_E5M2", "I8", "I16", "I32", "I64", "U8", "U16", "U32", "U64",
          "BOOL"]


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def write(path: str, tensors: list, metadata: dict | None = None, header_override: bytes | None = None,
          align: int = 8) -> None:
    """tensors: [(name, dtype name, shape, raw bytes)] in file order."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = header_override if header_override is not None else json.dumps(header).encode()
    text += b" " * ((-len(text)) % align)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))
