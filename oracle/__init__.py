"""CPU oracle for Aljabr's quantized-inference hot path.

TEST INFRASTRUCTURE ONLY. This package is the checker for the HIP kernels and
the timed CPU baseline: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it. The product package
(``aljabr_amd``) never imports, loads or falls back to anything here.

The arithmetic lives in ``aljabr_oracle.c`` (a C restatement of the reference's
Java CPU path; each function cites the reference file:line it follows). This
module only binds it with ctypes and adds numpy conveniences.

Parity status of each oracle function (what pins it) is in ``aljabr_oracle.h``.
``orc_nf4_quantize`` is PARITY UNPINNED against the reference (its quantizer is
absent from the reference tree); it is pinned only by the decode(encode(w))
nearest-level invariant.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libaljabr_oracle.so")
_lib = None

QTYPE_Q4_0 = 2
QTYPE_Q8_0 = 8
QTYPE_Q4_K = 12
QTYPE_Q6_K = 14


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float


def _declare(L: ctypes.CDLL) -> None:
    sig = {
        "orc_f16_to_f32": (_F, [ctypes.c_uint16]),
        "orc_f32_to_f16_writer": (ctypes.c_uint16, [_F]),
        "orc_java_round": (_I32, [_F]),
        "orc_nf4_dequant": (None, [_P, _P, _I64, _I32, _P]),
        "orc_nf4_quantize": (None, [_P, _I64, _I32, _P, _P]),
        "orc_nf4_matvec": (None, [_P, _P, _I32, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_q4_0_quantize": (None, [_P, _I64, _P]),
        "orc_q8_0_quantize": (None, [_P, _I64, _P]),
        "orc_q4_0_dequant": (None, [_P, _I64, _P]),
        "orc_q8_0_dequant": (None, [_P, _I64, _P]),
        "orc_q4_0_dot_row": (_F, [_P, _I32, _P]),
        "orc_q8_0_dot_row": (_F, [_P, _I32, _P]),
        "orc_q4_0_matvec": (None, [_P, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_q8_0_matvec": (None, [_P, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_f16_matvec": (None, [_P, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_q4_k_dequant": (None, [_P, _I64, _P]),
        "orc_q6_k_dequant": (None, [_P, _I64, _P]),
        "orc_q4_k_dot_row": (_F, [_P, _I32, _P]),
        "orc_q6_k_dot_row": (_F, [_P, _I32, _P]),
        "orc_q4_k_matvec": (None, [_P, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_q6_k_matvec": (None, [_P, _P, _I64, _I64, _I32, _P, ctypes.c_int]),
        "orc_softcap": (None, [_P, _I64, _F]),
        "orc_attention_gqa": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                            ctypes.c_int, _P, ctypes.c_int]),
        "orc_fa4_attention": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F, _I32, _F, _I32,
                                             _P]),
        "orc_paged_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F,
                                               _I32, _I32, _I32, _F, _P]),
        "orc_rmsnorm": (None, [_P, _P, _P, _I32, _F]),
        "orc_rope": (None, [_P, _I32, _I32, _I32, _F]),
        "orc_swiglu": (None, [_P, _P, _P, _I32]),
        "orc_softmax": (None, [_P, _I32]),
        "orc_decode_attention": (None, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _F]),
        "orc_llama_decode": (_I32, [_P, _P, _I32, _I32, _P, _P, _P, _P, ctypes.c_int]),
        "orc_llama_decode_typed": (_I32, [_P, _P, _I32, _I32, _P, _P, _P, _P, ctypes.c_int]),
        "orc_step_decode": (_I32, [_P, _I32, _I32, _F, _I32, _P, _P, _P, ctypes.c_int]),
        "orc_fill_normal": (None, [ctypes.c_uint64, _F, _F, _P, _I64]),
        "orc_fill_uniform_int": (None, [ctypes.c_uint64, _I32, _P, _I64]),
        "orc_max_threads": (ctypes.c_int, []),
        "orc_round_f16": (_F, [_F]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def threads() -> int:
    return int(lib().orc_max_threads())


# ---- generator ------------------------------------------------------------

def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(n), dtype=np.float32)
    lib().orc_fill_normal(seed & ((1 << 64) - 1), mean, std, _ptr(out), out.size)
    return out


def uniform_int(seed: int, bound: int, n: int) -> np.ndarray:
    out = np.empty(int(n), dtype=np.int32)
    lib().orc_fill_uniform_int(seed & ((1 << 64) - 1), bound, _ptr(out), out.size)
    return out


# ---- scalars --------------------------------------------------------------

def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(h))


def f32_to_f16_writer(v: float) -> int:
    return int(lib().orc_f32_to_f16_writer(v))


def java_round(v: float) -> int:
    return int(lib().orc_java_round(v))


# ---- NF4 ------------------------------------------------------------------

NF4_TABLE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)


def nf4_quantize(w: np.ndarray, group: int = 64):
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    codes = np.empty((w.size + 1) // 2, dtype=np.uint8)
    absmax = np.empty((w.size + group - 1) // group, dtype=np.float32)
    lib().orc_nf4_quantize(_ptr(w), w.size, group, _ptr(codes), _ptr(absmax))
    return codes, absmax


def nf4_dequant(codes: np.ndarray, absmax: np.ndarray, numel: int, group: int = 64) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    absmax = np.ascontiguousarray(absmax, dtype=np.float32)
    out = np.empty(int(numel), dtype=np.float32)
    lib().orc_nf4_dequant(_ptr(codes), _ptr(absmax), out.size, group, _ptr(out))
    return out


def nf4_matvec(codes, absmax, x: np.ndarray, n: int, k: int, group: int = 64,
               nthreads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.size // k
    y = np.empty(m * n, dtype=np.float32)
    lib().orc_nf4_matvec(_ptr(np.ascontiguousarray(codes)), _ptr(np.ascontiguousarray(absmax)),
                         group, _ptr(x), n, k, m, _ptr(y), nthreads or threads())
    return y.reshape(m, n) if m > 1 else y


# ---- GGUF Q4_0 / Q8_0 -----------------------------------------------------

def block_bytes(qtype: int) -> int:
    return {QTYPE_Q4_0: 18, QTYPE_Q8_0: 34, QTYPE_Q4_K: 144, QTYPE_Q6_K: 210}[qtype]


def block_elems(qtype: int) -> int:
    return 256 if qtype in (QTYPE_Q4_K, QTYPE_Q6_K) else 32


_NAMES = {QTYPE_Q4_0: "q4_0", QTYPE_Q8_0: "q8_0", QTYPE_Q4_K: "q4_k", QTYPE_Q6_K: "q6_k"}


def _fn(qtype: int, what: str):
    return getattr(lib(), f"orc_{_NAMES[qtype]}_{what}")


def quantize(qtype: int, w: np.ndarray) -> np.ndarray:
    """GGUFWriter's Q4_0/Q8_0 encoders (the reference writes no K-quants)."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    out = np.empty(w.size // 32 * block_bytes(qtype), dtype=np.uint8)
    fn = lib().orc_q4_0_quantize if qtype == QTYPE_Q4_0 else lib().orc_q8_0_quantize
    fn(_ptr(w), w.size, _ptr(out))
    return out


def dequant(qtype: int, blocks: np.ndarray, numel: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(int(numel), dtype=np.float32)
    _fn(qtype, "dequant")(_ptr(blocks), out.size, _ptr(out))
    return out


def dot_row(qtype: int, row: np.ndarray, x: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(_fn(qtype, "dot_row")(_ptr(row), x.size, _ptr(x)))


def q_matvec(qtype: int, w: np.ndarray, x: np.ndarray, n: int, k: int,
             nthreads: int | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.size // k
    y = np.empty(m * n, dtype=np.float32)
    _fn(qtype, "matvec")(_ptr(np.ascontiguousarray(w)), _ptr(x), n, k, m, _ptr(y), nthreads or threads())
    return y.reshape(m, n) if m > 1 else y


def softcap(y: np.ndarray, cap: float) -> np.ndarray:
    y = np.array(y, dtype=np.float32, copy=True, order="C")
    lib().orc_softcap(_ptr(y), y.size, cap)
    return y


def random_k_blocks(qtype: int, nblocks: int, seed: int, scale: float = 1.0 / 256) -> np.ndarray:
    """Random Q4_K/Q6_K super-blocks: every code byte uniform, the fp16 block
    scales finite and of size ~`scale` (positive d; Q4_K dMin >= 0, as a
    quantizer writes them). Test and benchmark data, not a quantizer."""
    rng = np.random.default_rng(seed)
    bb = block_bytes(qtype)
    blocks = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    d = (rng.uniform(0.25, 1.0, size=nblocks) * scale).astype(np.float16).view(np.uint16)
    if qtype == QTYPE_Q4_K:
        dmin = (rng.uniform(0.0, 1.0, size=nblocks) * scale).astype(np.float16).view(np.uint16)
        blocks[:, 0] = d & 0xFF
        blocks[:, 1] = d >> 8
        blocks[:, 2] = dmin & 0xFF
        blocks[:, 3] = dmin >> 8
    else:
        blocks[:, 208] = d & 0xFF
        blocks[:, 209] = d >> 8
    return blocks.reshape(-1)


def f16_matvec(w_bits: np.ndarray, x: np.ndarray, n: int, k: int,
               nthreads: int | None = None) -> np.ndarray:
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.size // k
    y = np.empty(m * n, dtype=np.float32)
    lib().orc_f16_matvec(_ptr(w_bits), _ptr(x), n, k, m, _ptr(y), nthreads or threads())
    return y.reshape(m, n) if m > 1 else y


# ---- attention ------------------------------------------------------------

def attention_gqa(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask=None, causal=False,
                  nthreads: int | None = None) -> np.ndarray:
    """q [B,Hq,Sq,D], k/v [B,Hkv,Sk,D] float32 -> out [B,Hq,Sq,D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    mp = 0
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        mp = _ptr(mask)
    rc = lib().orc_attention_gqa(_ptr(q), _ptr(k), _ptr(v), mp or None, b, hq, hkv, sq, sk, d,
                                 int(bool(causal)), _ptr(out), nthreads or threads())
    if rc != 0:
        raise ValueError("GQA expects Q[B,Hq,Sq,D], K/V[B,Hkv,Sk,D] and a finite, non-NaN mask")
    return out


def paged_attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, block_table: np.ndarray,
                    context_lens: np.ndarray, scale: float, causal: bool = True, query_start_pos: int = 0,
                    sliding_window: int = 0, soft_cap: float = 0.0):
    """q [B,T,H,D], caches [blocks,Hkv,block_size,D] float32, block_table
    [B,max_blocks] int32, context_lens [B] int32 -> (status, out [B,T,H,D])."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    vc = np.ascontiguousarray(vc, dtype=np.float32)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    b, t, h, d = q.shape
    hkv, bs = kc.shape[1], kc.shape[2]
    out = np.full_like(q, np.nan)
    rc = lib().orc_paged_attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(bt), _ptr(cl), b, t, h, hkv, d, bs,
                                   bt.shape[1], scale, int(bool(causal)), query_start_pos, sliding_window,
                                   soft_cap, _ptr(out))
    return rc, out


def fa4_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool = True,
                  soft_cap: float = 0.0, window: int = 0) -> np.ndarray:
    """q [B,T,H,D], k/v [B,S,Hkv,D] float32 -> out [B,T,H,D] (FA4 prefill semantics)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, t, h, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    out = np.full_like(q, np.nan)
    rc = lib().orc_fa4_attention(_ptr(q), _ptr(k), _ptr(v), b, t, s, h, hkv, d, scale, int(bool(causal)), soft_cap,
                                 window, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_fa4_attention rejected the shape (status {rc})")
    return out


# ---- element-wise ---------------------------------------------------------

def gated_activation(gate: np.ndarray, up: np.ndarray, kind: int) -> np.ndarray:
    """The Metal FFN activation (MTLC/aljabr_metal_kernel_source.m:72-108;
    kind 2 = GELU, else SiLU, as aljabr_metal_matvec_api.m picks the pipeline):
    act(g) * up in fp32, with the cut-offs and non-finite -> 0."""
    g = np.asarray(gate, np.float32).astype(np.float64)
    if kind == 2:
        inner = 0.79788456 * (g + 0.044715 * g ** 3)
        act = np.where(g <= -10.0, 0.0, np.where(g >= 10.0, g, 0.5 * g * (1.0 + np.tanh(inner))))
    else:
        with np.errstate(over="ignore"):
            act = np.where(g <= -20.0, 0.0, np.where(g >= 20.0, g, g / (1.0 + np.exp(-g))))
    with np.errstate(invalid="ignore", over="ignore"):
        y = (act * np.asarray(up, np.float64)).astype(np.float32)
    return np.where(np.isfinite(y), y, np.float32(0.0))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = x.reshape(-1, w.size)
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        o = np.empty_like(row)
        lib().orc_rmsnorm(_ptr(row), _ptr(w), _ptr(o), w.size, eps)
        out[r] = o
    return out.reshape(x.shape)


def rope(x: np.ndarray, n_heads: int, head_dim: int, pos: int, base: float) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_rope(_ptr(y), n_heads, head_dim, pos, base)
    return y.reshape(np.shape(x))


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    up = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    out = np.empty_like(gate)
    lib().orc_swiglu(_ptr(gate), _ptr(up), _ptr(out), gate.size)
    return out


def softmax(a: np.ndarray) -> np.ndarray:
    y = np.array(a, dtype=np.float32, copy=True).reshape(-1)
    lib().orc_softmax(_ptr(y), y.size)
    return y


def decode_attention(query: np.ndarray, keys: np.ndarray, values: np.ndarray, cache_head_stride: int,
                     kv_heads: int, query_heads: int, head_dim: int, sequence_length: int,
                     start_position: int, scale: float) -> np.ndarray:
    """The decode runner's attention (orc_decode_attention): keys/values are
    position-major [position][cache_head_stride] flat arrays."""
    q = np.ascontiguousarray(query, np.float32).reshape(-1)
    k = np.ascontiguousarray(keys, np.float32).reshape(-1)
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    out = np.empty(query_heads * head_dim, np.float32)
    scores = np.empty(max(sequence_length - start_position, 1), np.float32)
    lib().orc_decode_attention(_ptr(q), _ptr(out), _ptr(scores), _ptr(k), _ptr(v), cache_head_stride, kv_heads,
                               query_heads, head_dim, sequence_length, start_position, scale)
    return out


# ---- Llama-shaped decode step ---------------------------------------------

class _LlamaCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "layers", "dim", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab", "max_seq",
        "nf4_group", "kv_f16")] + [("rope_base", ctypes.c_float), ("eps", ctypes.c_float)]


_VP = ctypes.c_void_p


class _LlamaWeights(ctypes.Structure):
    _fields_ = [("tok_embed", _VP), ("attn_norm", _VP), ("ffn_norm", _VP),
                ("wq", _VP), ("wk", _VP), ("wv", _VP), ("wo", _VP),
                ("wq_s", _VP), ("wk_s", _VP), ("wv_s", _VP), ("wo_s", _VP),
                ("w_gate", _VP), ("w_up", _VP), ("w_down", _VP),
                ("w_gate_s", _VP), ("w_up_s", _VP), ("w_down_s", _VP),
                ("out_norm", _VP), ("lm_head", _VP)]


class LlamaOracle:
    """Single-sequence decode with the oracle (GgufDecodePass restated).

    ``weights`` maps names to numpy arrays: tok_embed [vocab*dim] f32,
    lm_head [vocab*dim] u16 (fp16 bits), out_norm [dim] f32 and per-layer lists
    attn_norm, ffn_norm (f32) and wq/wk/wv/wo/w_gate/w_up/w_down (codes u8)
    with their *_s absmax (f32)."""

    LAYER_KEYS = ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "wq_s", "wk_s", "wv_s", "wo_s",
                  "w_gate", "w_up", "w_down", "w_gate_s", "w_up_s", "w_down_s")

    def __init__(self, cfg: dict, weights: dict, kv_f16: bool = True):
        self.cfg = _LlamaCfg(cfg["layers"], cfg["dim"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                             cfg["head_dim"], cfg["vocab"], cfg["max_seq"], cfg["nf4_block"], int(kv_f16),
                             cfg["rope_base"], cfg["eps"])
        self._keep = []
        w = _LlamaWeights()
        for key in ("tok_embed", "out_norm", "lm_head"):
            arr = np.ascontiguousarray(weights[key])
            self._keep.append(arr)
            setattr(w, key, arr.ctypes.data)
        for key in self.LAYER_KEYS:
            arrs = [np.ascontiguousarray(a) for a in weights[key]]
            self._keep.extend(arrs)
            table = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
            self._keep.append(table)
            setattr(w, key, ctypes.cast(table, ctypes.c_void_p).value)
        self.weights = w
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        self.k_cache = np.zeros(cfg["layers"] * cfg["max_seq"] * kvd, np.float32)
        self.v_cache = np.zeros_like(self.k_cache)
        self.dim, self.vocab = cfg["dim"], cfg["vocab"]

    def decode(self, token: int, pos: int, nthreads: int | None = None):
        logits = np.empty(self.vocab, np.float32)
        hidden = np.empty(self.dim, np.float32)
        nxt = lib().orc_llama_decode(ctypes.byref(self.cfg), ctypes.byref(self.weights), token, pos,
                                     _ptr(self.k_cache), _ptr(self.v_cache), _ptr(logits), _ptr(hidden),
                                     nthreads or threads())
        return int(nxt), logits, hidden


class _Tensor(ctypes.Structure):
    _fields_ = [("data", _VP), ("absmax", _VP), ("type", ctypes.c_int32), ("group", ctypes.c_int32)]


class _LlamaTyped(ctypes.Structure):
    _fields_ = [("tok_embed", _Tensor), ("attn_norm", _VP), ("ffn_norm", _VP),
                ("wq", _VP), ("wk", _VP), ("wv", _VP), ("wo", _VP),
                ("w_gate", _VP), ("w_up", _VP), ("w_down", _VP),
                ("out_norm", _VP), ("lm_head", _Tensor)]


class TypedLlamaOracle:
    """Single-sequence decode over per-tensor types (GgufDecodePass over GGUF
    GgmlTypes, restated): ``weights`` maps tok_embed, lm_head and the
    per-layer lists wq, wk, wv, wo, w_gate, w_up, w_down to (type, array)
    pairs (type ids as ALJABR_ROCM_TYPE_*: 0 F32, 1 F16 (uint16 bits), 2 Q4_0,
    8 Q8_0, 12 Q4_K, 14 Q6_K (bytes)), or (100, codes, absmax) triples for
    NF4 with block cfg["nf4_block"], and attn_norm, ffn_norm (lists) and
    out_norm to fp32 arrays."""

    MATS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")

    def __init__(self, cfg: dict, weights: dict, kv_f16: bool = True):
        self.cfg = _LlamaCfg(cfg["layers"], cfg["dim"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                             cfg["head_dim"], cfg["vocab"], cfg["max_seq"], cfg.get("nf4_block", 64), int(kv_f16),
                             cfg["rope_base"], cfg["eps"])
        self._keep = []

        def tensor(pair):
            if len(pair) == 3:                       # NF4: (100, codes, absmax), block cfg["nf4_block"]
                t, arr, absmax = pair
                absmax = np.ascontiguousarray(absmax, np.float32)
                self._keep.append(absmax)
                arr = np.ascontiguousarray(arr)
                self._keep.append(arr)
                return _Tensor(arr.ctypes.data, absmax.ctypes.data, t, cfg.get("nf4_block", 64))
            t, arr = pair
            arr = np.ascontiguousarray(arr)
            self._keep.append(arr)
            return _Tensor(arr.ctypes.data, None, t, 0)

        def table(arrs, ctype):
            tab = (ctype * len(arrs))(*arrs)
            self._keep.append(tab)
            return ctypes.cast(tab, ctypes.c_void_p).value

        w = _LlamaTyped()
        w.tok_embed = tensor(weights["tok_embed"])
        w.lm_head = tensor(weights["lm_head"])
        norm = np.ascontiguousarray(weights["out_norm"], np.float32)
        self._keep.append(norm)
        w.out_norm = norm.ctypes.data
        for key in ("attn_norm", "ffn_norm"):
            arrs = [np.ascontiguousarray(a, np.float32) for a in weights[key]]
            self._keep.extend(arrs)
            setattr(w, key, table([a.ctypes.data for a in arrs], ctypes.c_void_p))
        for key in self.MATS:
            setattr(w, key, table([tensor(p) for p in weights[key]], _Tensor))
        self.weights = w
        kvd = cfg["n_kv_heads"] * cfg["head_dim"]
        self.k_cache = np.zeros(cfg["layers"] * cfg["max_seq"] * kvd, np.float32)
        self.v_cache = np.zeros_like(self.k_cache)
        self.dim, self.vocab = cfg["dim"], cfg["vocab"]

    def decode(self, token: int, pos: int, nthreads: int | None = None):
        logits = np.empty(self.vocab, np.float32)
        hidden = np.empty(self.dim, np.float32)
        nxt = lib().orc_llama_decode_typed(ctypes.byref(self.cfg), ctypes.byref(self.weights), token, pos,
                                           _ptr(self.k_cache), _ptr(self.v_cache), _ptr(logits), _ptr(hidden),
                                           nthreads or threads())
        return int(nxt), logits, hidden


# ---- Metal whole-step decode ----------------------------------------------

class _StepLayer(ctypes.Structure):
    _fields_ = [(n, _Tensor) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] + \
        [(n, _I32) for n in ("kv_layer", "n0", "n1", "n2", "wo_k", "wo_n", "ffn", "n_heads", "n_kv_heads",
                             "head_dim")] + \
        [("freq_base", _F), ("is_swa", _I32), ("out_scale", _F), ("attn_scale", _F)] + \
        [(n, _I32) for n in ("has_post_attn_norm", "has_post_ffn_norm", "has_q_norm", "has_k_norm",
                             "has_unit_v_norm")] + \
        [("rope_freqs", _P), ("rope_freqs_len", _I32)]


class _StepModel(ctypes.Structure):
    _fields_ = [("layers", _I32), ("layer", ctypes.POINTER(_StepLayer)), ("norm", _P * 6),
                ("k_cache", _P), ("v_cache", _P), ("kv_stride", _P), ("out_norm", _P), ("out_w", _Tensor),
                ("out_k", _I32), ("out_n", _I32), ("cap", _F), ("embd", _Tensor), ("embd_rows", _I32),
                ("embd_scale", _F), ("activation", _I32)]


STEP_FLAGS = ("has_post_attn_norm", "has_post_ffn_norm", "has_q_norm", "has_k_norm", "has_unit_v_norm")


class StepOracle:
    """The Metal whole-step decode restated (orc_step_decode). ``model`` is a
    dict: ``dim``, ``max_seq``, ``activation`` (1 SiLU, 2 GELU), ``layers``
    (a list of dicts with (type, array) pairs for wq, wk, wv, wo, gate, up,
    down -- wk / wv may be None --, kv_layer, n_heads, n_kv_heads, head_dim,
    ffn, freq_base, is_swa, out_scale, attn_scale, the has_* flags and
    rope_freqs (array or None)), ``norm`` (six flat fp32 arrays or None, the
    norm slots), ``out_norm``, ``out_w`` ((type, array) or None), ``vocab``,
    ``cap``, ``embd`` ((type, array) or None) and ``embd_scale``."""

    def __init__(self, model: dict):
        self._keep = []
        dim = model["dim"]
        n = len(model["layers"])

        def tensor(pair):
            if pair is None:
                return _Tensor(None, None, 0, 0)
            t, arr = pair
            arr = np.ascontiguousarray(arr)
            self._keep.append(arr)
            return _Tensor(arr.ctypes.data, None, t, 0)

        def keep(a, dtype=np.float32):
            a = np.ascontiguousarray(a, dtype)
            self._keep.append(a)
            return a

        layers = (_StepLayer * n)()
        self.k_cache, self.v_cache, strides = [], [], []
        for i, c in enumerate(model["layers"]):
            L = layers[i]
            for key in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
                setattr(L, key, tensor(c.get(key)))
            nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
            L.kv_layer = c.get("kv_layer", i)
            L.n0, L.n1, L.n2 = nh * hd, nkv * hd, nkv * hd
            L.wo_k, L.wo_n, L.ffn = nh * hd, dim, c["ffn"]
            L.n_heads, L.n_kv_heads, L.head_dim = nh, nkv, hd
            L.freq_base = c.get("freq_base", 10000.0)
            L.is_swa = int(c.get("is_swa", 0))
            L.out_scale = c.get("out_scale", 1.0)
            L.attn_scale = c.get("attn_scale", 0.0)
            for f in STEP_FLAGS:
                setattr(L, f, int(c.get(f, 0)))
            if c.get("rope_freqs") is not None:
                rf = keep(c["rope_freqs"])
                L.rope_freqs, L.rope_freqs_len = rf.ctypes.data, rf.size
            stride = nkv * hd
            strides.append(stride)
            kc = keep(np.zeros(model["max_seq"] * stride))
            vc = keep(np.zeros(model["max_seq"] * stride))
            self.k_cache.append(kc)
            self.v_cache.append(vc)
        self._keep.append(layers)
        m = _StepModel()
        m.layers = n
        m.layer = layers
        for slot in range(6):
            arr = model["norm"][slot]
            m.norm[slot] = keep(arr).ctypes.data if arr is not None else None
        kp = (_P * n)(*[a.ctypes.data for a in self.k_cache])
        vp = (_P * n)(*[a.ctypes.data for a in self.v_cache])
        st = (_I32 * n)(*strides)
        self._keep += [kp, vp, st]
        m.k_cache, m.v_cache, m.kv_stride = ctypes.addressof(kp), ctypes.addressof(vp), ctypes.addressof(st)
        if model.get("out_w") is not None:
            m.out_norm = keep(model["out_norm"]).ctypes.data
            m.out_w = tensor(model["out_w"])
            m.out_k, m.out_n = dim, model["vocab"]
        m.cap = model.get("cap", 0.0)
        m.embd = tensor(model.get("embd"))
        m.embd_rows = model.get("vocab", 0)
        m.embd_scale = model.get("embd_scale", 1.0)
        m.activation = model.get("activation", 2)
        self.model = m
        self.dim, self.vocab = dim, model.get("vocab", 0)

    def decode(self, pos: int, window: int = 0, eps: float = 1e-6, token: int = -1, x_in=None,
               nthreads: int | None = None):
        """One position: returns (status or greedy token, residual x, logits)."""
        x = np.empty(self.dim, np.float32)
        logits = np.zeros(max(self.vocab, 1), np.float32)
        xin = np.ascontiguousarray(x_in, np.float32) if x_in is not None else None
        rc = lib().orc_step_decode(ctypes.byref(self.model), pos, window, eps, token,
                                   xin.ctypes.data if xin is not None else None, _ptr(x), _ptr(logits),
                                   nthreads or threads())
        return int(rc), x, logits
