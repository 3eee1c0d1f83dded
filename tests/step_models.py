"""Small models for the registered whole-step decode (the Metal ABI's
register_decode_layer / decode_step contract), shared by the oracle pins and
the GPU parity tests.

``gemma_like`` exercises every per-layer feature the reference's step carries
(MTLC/aljabr_metal_matvec_api.m:3574-4083): Q/K head norms, a unit V norm,
post-attention and post-FFN norms, RoPE frequency divisors, sliding-window
layers, a K-as-V layer (wk without wv), a layer that shares an earlier
layer's KV cache (neither wk nor wv), output scales, an explicit attention
scale and a logit softcap. ``llama_like`` turns all of them off.
"""
from __future__ import annotations

import numpy as np

DIM, FFN, NH, NKV, HD, VOCAB = 64, 96, 4, 2, 16, 50


def _w(oracle, seed, n, k, std=0.15):
    return oracle.normal(seed, n * k, 0.0, std)


def _norm_rows(oracle, seed, rows, n):
    return (1.0 + 0.1 * oracle.normal(seed, rows * n)).astype(np.float32)


def _layer(oracle, seed, *, wk=True, wv=True, **kw):
    qd, kvd = NH * HD, NKV * HD
    c = dict(wq=(0, _w(oracle, seed + 1, qd, DIM)),
             wk=(0, _w(oracle, seed + 2, kvd, DIM)) if wk else None,
             wv=(0, _w(oracle, seed + 3, kvd, DIM)) if wv else None,
             wo=(0, _w(oracle, seed + 4, DIM, qd)),
             gate=(0, _w(oracle, seed + 5, FFN, DIM)),
             up=(0, _w(oracle, seed + 6, FFN, DIM)),
             down=(0, _w(oracle, seed + 7, DIM, FFN)),
             n_heads=NH, n_kv_heads=NKV, head_dim=HD, ffn=FFN, freq_base=10000.0)
    c.update(kw)
    return c


def llama_like(oracle, seed=100, layers=2, max_seq=16, activation=1):
    model = dict(dim=DIM, max_seq=max_seq, activation=activation, vocab=VOCAB, cap=0.0, embd_scale=1.0,
                 layers=[_layer(oracle, seed + 10 * l) for l in range(layers)])
    norm = [None] * 6
    norm[3] = _norm_rows(oracle, seed + 1000, layers, DIM)   # attention norm
    norm[1] = _norm_rows(oracle, seed + 1001, layers, DIM)   # FFN norm
    model["norm"] = norm
    model["out_norm"] = _norm_rows(oracle, seed + 1002, 1, DIM)
    model["out_w"] = (0, _w(oracle, seed + 1003, VOCAB, DIM, 0.1))
    model["embd"] = (0, oracle.normal(seed + 1004, VOCAB * DIM))
    return model


def gemma_like(oracle, seed=300, max_seq=24, window=5):
    """Four layers: 0 sliding-window with every norm and RoPE divisors; 1
    global, K-as-V with a unit V norm and an output scale; 2 sliding-window
    sharing layer 0's cache; 3 global with an explicit attention scale."""
    freqs = np.where(np.arange(HD // 2) % 3 == 0, 1.0, 1.0 + np.arange(HD // 2) / 4.0).astype(np.float32)
    freqs[5] = -1.0                                  # not positive: treated as 1
    layers = [
        _layer(oracle, seed, is_swa=1, has_q_norm=1, has_k_norm=1, has_post_attn_norm=1, has_post_ffn_norm=1,
               rope_freqs=freqs, freq_base=10000.0),
        _layer(oracle, seed + 10, wv=False, has_unit_v_norm=1, out_scale=0.75, freq_base=500000.0,
               has_post_ffn_norm=1),
        _layer(oracle, seed + 20, wk=False, wv=False, kv_layer=0, is_swa=1, has_q_norm=1, has_post_attn_norm=1,
               rope_freqs=freqs),
        _layer(oracle, seed + 30, attn_scale=0.2, out_scale=1.25),
    ]
    n = len(layers)
    norm = [_norm_rows(oracle, seed + 1000 + s, n, DIM) for s in range(4)]
    norm += [_norm_rows(oracle, seed + 1010 + s, n, HD) for s in range(2)]
    return dict(dim=DIM, max_seq=max_seq, activation=2, vocab=VOCAB, cap=3.0, embd_scale=1.5, layers=layers,
                norm=norm, out_norm=_norm_rows(oracle, seed + 1020, 1, DIM),
                out_w=(0, _w(oracle, seed + 1021, VOCAB, DIM, 0.1)),
                embd=(0, oracle.normal(seed + 1022, VOCAB * DIM))), window


# ---- an independent full-sequence forward ----------------------------------

def forward(model, inputs, window: int, eps: float, mistake: str = ""):
    """Causal forward over a whole sequence at once in float64: inputs are the
    layer-0 residual rows [T, dim]; returns logits [T, vocab] and the final
    residual rows [T, dim]. Written from the step's equations, not from the
    oracle's loop: every layer works on all positions as matrices, keys are
    chosen by a mask, and shared-cache layers read the owner's K/V arrays."""
    x = np.asarray(inputs, np.float64).copy()
    n = x.shape[0]
    layers = model["layers"]
    kv = {}

    def dense(pair, rows, cols):
        return np.asarray(pair[1], np.float64).reshape(rows, cols)

    def rms(v, w=None):
        r = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps)
        return r * w if w is not None else r

    def rope(v, heads, hd, base, freqs):
        half = hd // 2
        inv = base ** (-2.0 * np.arange(half) / hd)
        if freqs is not None:
            ff = np.asarray(freqs, np.float64)
            if mistake == "freq_factor_multiplied":
                inv = inv * np.where(ff > 0, ff, 1.0)
            else:
                inv = inv / np.where(ff > 0, ff, 1.0)
        ang = np.arange(n, dtype=np.float64)[:, None] * inv[None, :]
        cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        v = v.reshape(n, heads, hd).copy()
        a, b = v[..., :half].copy(), v[..., half:].copy()
        v[..., :half] = a * cos - b * sin
        v[..., half:] = a * sin + b * cos
        return v

    def gated(g, u):
        if model["activation"] == 2:
            act = np.where(g <= -10, 0.0, np.where(g >= 10, g, 0.5 * g * (1 + np.tanh(
                0.79788456 * (g + 0.044715 * g ** 3)))))
        else:
            act = np.where(g <= -20, 0.0, np.where(g >= 20, g, g / (1 + np.exp(-g))))
        return act * u

    dim = model["dim"]
    for l, c in enumerate(layers):
        nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        norm = model["norm"]
        xn = rms(x, norm[3].reshape(-1, dim)[l])
        q = xn @ dense(c["wq"], nh * hd, dim).T
        if c.get("has_q_norm"):
            q = rms(q.reshape(n, nh, hd), norm[4].reshape(-1, hd)[l]).reshape(n, -1)
        q = rope(q, nh, hd, c["freq_base"], c.get("rope_freqs"))
        if c.get("wk") is not None:
            k_raw = xn @ dense(c["wk"], nkv * hd, dim).T
            v = xn @ dense(c["wv"], nkv * hd, dim).T if c.get("wv") is not None else k_raw.copy()
            k = k_raw
            if c.get("has_k_norm"):
                k = rms(k.reshape(n, nkv, hd), norm[5].reshape(-1, hd)[l]).reshape(n, -1)
            k = rope(k, nkv, hd, c["freq_base"], c.get("rope_freqs"))
            if c.get("wv") is None and mistake == "kv_as_v_after_rope":
                v = k.reshape(n, -1).copy()
            v = v.reshape(n, nkv, hd)
            if c.get("has_unit_v_norm") and mistake != "unit_v_norm_missing":
                v = rms(v)
            kv[l] = (k, v)
        owner = c.get("kv_layer", l)
        if mistake == "shared_kv_wrong_owner" and c.get("wk") is None:
            owner = 1
        k, v = kv[owner]
        scale = c.get("attn_scale", 0.0)
        if scale <= 0:
            scale = 1.0 if (c.get("has_q_norm") or c.get("has_k_norm")) else 1.0 / np.sqrt(hd)
        i, j = np.arange(n)[:, None], np.arange(n)[None, :]
        mask = j <= i
        if c.get("is_swa") and window > 0:
            lim = window + (1 if mistake == "window_off_by_one" else 0)
            mask &= j > i - lim
        att = np.zeros((n, nh, hd))
        for h in range(nh):
            g = h // (nh // nkv)
            sc = np.where(mask, q[:, h, :] @ k[:, g, :].T * scale, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            att[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ v[:, g, :]
        o = att.reshape(n, nh * hd) @ dense(c["wo"], dim, nh * hd).T
        if c.get("has_post_attn_norm"):
            if mistake == "post_norm_after_residual":
                x = rms(x + o, norm[0].reshape(-1, dim)[l])
            else:
                x = x + rms(o, norm[0].reshape(-1, dim)[l])
        else:
            x = x + o
        xn = rms(x, norm[1].reshape(-1, dim)[l])
        hb = gated(xn @ dense(c["gate"], c["ffn"], dim).T, xn @ dense(c["up"], c["ffn"], dim).T)
        d = hb @ dense(c["down"], dim, c["ffn"]).T
        if c.get("has_post_ffn_norm"):
            d = rms(d, norm[2].reshape(-1, dim)[l])
        s = c.get("out_scale", 1.0)
        if s > 0 and s != 1.0:
            x = x + d * s if mistake == "out_scale_on_branch" else (x + d) * s
        else:
            x = x + d
    logits = rms(x, np.asarray(model["out_norm"], np.float64)) @ dense(model["out_w"], model["vocab"], dim).T
    cap = model.get("cap", 0.0)
    if cap > 0 and mistake != "softcap_missing":
        logits = cap * np.tanh(logits / cap)
    return logits, x


def token_inputs(model, tokens):
    """Layer-0 residual rows of a token sequence: embedding rows times the
    embedding scale."""
    emb = np.asarray(model["embd"][1], np.float32).reshape(-1, model["dim"])
    return emb[np.asarray(tokens)] * np.float32(model.get("embd_scale", 1.0))
