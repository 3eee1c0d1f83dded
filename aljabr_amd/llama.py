"""Host-side driver of the device-resident Llama decode step.

The caller above the C ABI: it owns the weight buffers (torch device memory
as plumbing), builds the ``aljabr_rocm_llama_weights`` pointer tables and
runs ``aljabr_rocm_llama_decode``, as GgufDecodePass drives one decode
position per call (engine/gguf/aljabr-gguf-java/.../GgufDecodePass.java:183-592).
Random-init weights are drawn on the device (N(0, 0.02) for projections) and
quantized there by ``aljabr_rocm_quantize``; host numpy weights can be
uploaded instead for parity checks.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import abi

LLAMA3_8B = dict(layers=32, dim=4096, ffn=14336, n_heads=32, n_kv_heads=8, head_dim=128, vocab=128256,
                 nf4_block=64, rope_base=500000.0, eps=1e-5)

PROJ = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


def proj_shapes(cfg: dict) -> dict:
    """[out, in] of every per-layer projection."""
    d, hd = cfg["dim"], cfg["head_dim"]
    qd, kvd = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    return {"wq": (qd, d), "wk": (kvd, d), "wv": (kvd, d), "wo": (d, qd),
            "w_gate": (cfg["ffn"], d), "w_up": (cfg["ffn"], d), "w_down": (d, cfg["ffn"])}


def nf4_quantize_device(w, block: int):
    """fp32 device tensor -> (codes uint8, absmax f32) device tensors via the C ABI."""
    import torch
    n = w.numel()
    codes = torch.empty((n + 1) // 2, dtype=torch.uint8, device=w.device)
    absmax = torch.empty((n + block - 1) // block, dtype=torch.float32, device=w.device)
    torch.cuda.synchronize()
    abi.call("aljabr_rocm_quantize", codes.data_ptr(), absmax.data_ptr(), w.data_ptr(), n, abi.TYPE_NF4, block)
    # The caller may free `w` next: wait for the encoder in stream-ordered mode too.
    abi.call("aljabr_rocm_synchronize")
    return codes, absmax


def random_weights(cfg: dict, seed: int = 0, device: str = "cuda:0") -> dict:
    """Random-init Llama-shaped weights on the device: NF4 projections from
    N(0, 0.02), fp32 norms near 1, fp32 N(0,1) embeddings, fp16 LM head."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    out = {k: [] for k in PROJ}
    out.update({k + "_s": [] for k in PROJ})
    out["attn_norm"], out["ffn_norm"] = [], []
    shapes = proj_shapes(cfg)
    for _ in range(cfg["layers"]):
        for name in PROJ:
            n, k = shapes[name]
            w = torch.randn(n * k, generator=g, device=device, dtype=torch.float32).mul_(0.02)
            c, a = nf4_quantize_device(w, cfg["nf4_block"])
            del w
            out[name].append(c)
            out[name + "_s"].append(a)
        for nm in ("attn_norm", "ffn_norm"):
            out[nm].append(1.0 + 0.1 * torch.randn(cfg["dim"], generator=g, device=device))
    out["out_norm"] = 1.0 + 0.1 * torch.randn(cfg["dim"], generator=g, device=device)
    out["tok_embed"] = torch.randn(cfg["vocab"] * cfg["dim"], generator=g, device=device)
    out["lm_head"] = (0.02 * torch.randn(cfg["vocab"] * cfg["dim"], generator=g, device=device)).half()
    torch.cuda.synchronize()
    return out


def upload_weights(host: dict, device: str = "cuda:0") -> dict:
    """Host numpy weights (oracle.LlamaOracle layout) -> device tensors."""
    import torch

    def put(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            a = a.view(np.int16)
        return torch.from_numpy(a).to(device)

    out = {}
    for key, val in host.items():
        out[key] = [put(a) for a in val] if isinstance(val, list) else put(val)
    torch.cuda.synchronize()
    return out


class DeviceLlama:
    """One decode session (KV cache + activations) over caller-owned weights."""

    def __init__(self, cfg: dict, weights: dict, max_batch: int, max_seq: int):
        lib = abi.load()
        self.cfg = dict(cfg)
        self.weights = weights   # keeps the device buffers alive
        c = abi.LlamaConfig(cfg["layers"], cfg["dim"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                            cfg["head_dim"], cfg["vocab"], max_seq, cfg["nf4_block"], max_batch,
                            cfg["rope_base"], cfg["eps"])
        w = abi.LlamaWeights()
        self._tables = []
        for key in ("tok_embed", "out_norm", "lm_head"):
            setattr(w, key, weights[key].data_ptr())
        for key, field in [("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm")] + \
                [(n, n) for n in PROJ] + [(n + "_s", n + "_absmax") for n in PROJ]:
            ptrs = (ctypes.c_void_p * cfg["layers"])(*[t.data_ptr() for t in weights[key]])
            self._tables.append(ptrs)
            setattr(w, field, ctypes.cast(ptrs, ctypes.POINTER(ctypes.c_void_p)))
        handle = ctypes.c_void_p()
        abi.check(lib.aljabr_rocm_llama_create(ctypes.byref(c), ctypes.byref(w), ctypes.byref(handle)),
                  "aljabr_rocm_llama_create")
        self.handle = handle
        self.max_batch, self.max_seq = max_batch, max_seq

    @classmethod
    def _wrap(cls, handle, cfg: dict, max_batch: int, max_seq: int, keep):
        self = cls.__new__(cls)
        self.cfg, self.weights, self._tables = dict(cfg), keep, []
        self.handle, self.max_batch, self.max_seq = handle, max_batch, max_seq
        return self

    @classmethod
    def from_gguf(cls, path: str, max_batch: int, max_seq: int = 0):
        """A session over a Llama-family GGUF file (aljabr_rocm_llama_create_gguf):
        the library uploads the file's tensors once and owns them."""
        lib = abi.load()
        handle = ctypes.c_void_p()
        abi.check(lib.aljabr_rocm_llama_create_gguf(path.encode(), max_batch, max_seq, ctypes.byref(handle)),
                  "aljabr_rocm_llama_create_gguf")
        c = abi.LlamaConfig()
        abi.check(lib.aljabr_rocm_llama_config_get(handle, ctypes.byref(c)), "aljabr_rocm_llama_config_get")
        cfg = {name: getattr(c, name) for name, _ in abi.LlamaConfig._fields_}
        return cls._wrap(handle, cfg, max_batch, c.max_seq, None)

    @classmethod
    def from_safetensors(cls, path: str, cfg: dict, max_batch: int, max_seq: int):
        """A session over a safetensors file with Hugging Face Llama names and
        NF4 or dense projections (aljabr_rocm_llama_create_safetensors); the
        architecture comes from `cfg` (layers, dim, ffn, n_heads, n_kv_heads,
        head_dim, vocab, rope_base, eps) and the library owns the weights."""
        lib = abi.load()
        c = abi.LlamaConfig(cfg["layers"], cfg["dim"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                            cfg["head_dim"], cfg["vocab"], max_seq, 128, max_batch, cfg["rope_base"], cfg["eps"])
        handle = ctypes.c_void_p()
        abi.check(lib.aljabr_rocm_llama_create_safetensors(path.encode(), ctypes.byref(c), ctypes.byref(handle)),
                  "aljabr_rocm_llama_create_safetensors")
        abi.check(lib.aljabr_rocm_llama_config_get(handle, ctypes.byref(c)), "aljabr_rocm_llama_config_get")
        full = {name: getattr(c, name) for name, _ in abi.LlamaConfig._fields_}
        return cls._wrap(handle, full, max_batch, max_seq, None)

    @classmethod
    def typed(cls, cfg: dict, weights: dict, max_batch: int, max_seq: int):
        """A session over typed device weights (aljabr_rocm_llama_create_typed):
        tok_embed and lm_head are (type, tensor) pairs, the PROJ lists hold
        (type, tensor) or, for NF4, (TYPE_NF4, (codes, absmax)); attn_norm and
        ffn_norm are lists of fp32 tensors, out_norm an fp32 tensor."""
        lib = abi.load()
        c = abi.LlamaConfig(cfg["layers"], cfg["dim"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                            cfg["head_dim"], cfg["vocab"], max_seq, cfg.get("nf4_block", 64), max_batch,
                            cfg["rope_base"], cfg["eps"])
        keep = []

        def tensor(pair):
            t, data = pair
            if t == abi.TYPE_NF4:
                codes, absmax = data
                return abi.Tensor(codes.data_ptr(), absmax.data_ptr(), t, cfg.get("nf4_block", 64))
            return abi.Tensor(data.data_ptr(), None, t, 0)

        w = abi.LlamaTensors()
        w.tok_embed = tensor(weights["tok_embed"])
        w.lm_head = tensor(weights["lm_head"])
        w.out_norm = weights["out_norm"].data_ptr()
        for key in ("attn_norm", "ffn_norm"):
            tab = (ctypes.c_void_p * cfg["layers"])(*[t.data_ptr() for t in weights[key]])
            keep.append(tab)
            setattr(w, key, ctypes.cast(tab, ctypes.POINTER(ctypes.c_void_p)))
        for key in PROJ:
            tab = (abi.Tensor * cfg["layers"])(*[tensor(p) for p in weights[key]])
            keep.append(tab)
            setattr(w, key, ctypes.cast(tab, ctypes.POINTER(abi.Tensor)))
        handle = ctypes.c_void_p()
        abi.check(lib.aljabr_rocm_llama_create_typed(ctypes.byref(c), ctypes.byref(w), ctypes.byref(handle)),
                  "aljabr_rocm_llama_create_typed")
        return cls._wrap(handle, dict(cfg, max_seq=max_seq), max_batch, max_seq, (weights, keep))

    def decode(self, tokens, positions, batch: int, logits=None, next_tokens=None):
        """tokens/positions: int32 device tensors; returns next_tokens (int32 device)."""
        import torch
        if next_tokens is None:
            next_tokens = torch.empty(batch, dtype=torch.int32, device=tokens.device)
        abi.call("aljabr_rocm_llama_decode", self.handle, tokens.data_ptr(), positions.data_ptr(), batch,
                 logits.data_ptr() if logits is not None else None, next_tokens.data_ptr())
        return next_tokens

    def decode_graph(self, tokens, positions, batch: int, logits=None, next_tokens=None):
        """decode() replayed from the session's captured HIP graph of the step."""
        import torch
        if next_tokens is None:
            next_tokens = torch.empty(batch, dtype=torch.int32, device=tokens.device)
        abi.call("aljabr_rocm_llama_decode_graph", self.handle, tokens.data_ptr(), positions.data_ptr(), batch,
                 logits.data_ptr() if logits is not None else None, next_tokens.data_ptr())
        return next_tokens

    def decode_profile(self, tokens, positions, batch: int, logits=None, next_tokens=None):
        """One decode step with per-launch-group device times; returns
        (next_tokens, [{"name", "launches", "us", "bytes"}, ...])."""
        import torch
        if next_tokens is None:
            next_tokens = torch.empty(batch, dtype=torch.int32, device=tokens.device)
        cap = 64
        stats = (abi.KernelStat * cap)()
        count = ctypes.c_int(0)
        abi.call("aljabr_rocm_llama_decode_profile", self.handle, tokens.data_ptr(), positions.data_ptr(), batch,
                 logits.data_ptr() if logits is not None else None, next_tokens.data_ptr(), stats, cap,
                 ctypes.byref(count))
        groups = [{"name": stats[i].name.decode(), "launches": stats[i].launches, "us": stats[i].us,
                   "bytes": stats[i].bytes} for i in range(count.value)]
        return next_tokens, groups

    def hidden_ptr(self) -> int:
        p = ctypes.c_void_p()
        abi.call("aljabr_rocm_llama_hidden", self.handle, ctypes.byref(p))
        return p.value

    def kv_cache_ptrs(self):
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        abi.call("aljabr_rocm_llama_kv_cache", self.handle, ctypes.byref(k), ctypes.byref(v))
        return k.value, v.value

    def kv_cache_elems(self) -> int:
        c = self.cfg
        return c["layers"] * self.max_batch * c["n_kv_heads"] * self.max_seq * c["head_dim"]

    def close(self):
        if self.handle:
            abi.call("aljabr_rocm_llama_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
