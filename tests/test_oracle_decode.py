"""Pins of the decode-step oracle (CPU only, no GPU).

The decode runner's attention (orc_decode_attention) against the reference's
own known answers (GgufDecodeAttentionExecutionTest.java:15-66) and against
the dense attention oracle; the whole step (orc_llama_decode_typed, fed one
token per position) against an independent full-sequence causal forward
written here in float64 numpy from the equations of GgufDecodePass.java:297-505
(RMSNorm GGUFVectorOps.java:211-234, split-half RoPE :383-440, softmax
:302-317, SwiGLU :333-338); and closed forms. Mistakes planted in the numpy
forward (a dropped residual, interleaved RoPE pairs, a wrong GQA head map, an
off-by-one causal window, gate and up swapped) must each move the result far
outside the tolerance, so the comparison would catch them in the oracle too.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import rel_l2

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))

CFG = dict(layers=2, dim=64, ffn=96, n_heads=4, n_kv_heads=2, head_dim=16, vocab=50, max_seq=16,
           rope_base=10000.0, eps=1e-5)
T = 12            # positions decoded


@pytest.mark.parametrize("case", KATS["decode_attention"], ids=lambda c: c["source"].split(":")[-1])
def test_decode_attention_known_answers(oracle, case):
    stride, kvh, qh, hd, seq, start, scale = case["args"]
    out = oracle.decode_attention(np.array(case["query"], np.float32), np.array(case["keys"], np.float32),
                                  np.array(case["values"], np.float32), stride, kvh, qh, hd, seq, start, scale)
    np.testing.assert_allclose(out, case["expected"], atol=case["tolerance"], rtol=0)


def test_decode_attention_matches_dense_oracle(oracle):
    """Position-major decode attention = the dense attentionGqa oracle (pinned
    by CpuBatchedAttentionTest) with Sq = 1 over the visible keys."""
    hq, hkv, d, s = 8, 2, 32, 37
    q = oracle.normal(1, hq * d)
    k = oracle.normal(2, s * hkv * d)
    v = oracle.normal(3, s * hkv * d)
    scale = float(np.float32(1.0 / np.sqrt(d)))
    for start in (0, 5, 36):
        got = oracle.decode_attention(q, k, v, hkv * d, hkv, hq, d, s, start, scale)
        kd = k.reshape(s, hkv, d)[start:].transpose(1, 0, 2).reshape(1, hkv, s - start, d)
        vd = v.reshape(s, hkv, d)[start:].transpose(1, 0, 2).reshape(1, hkv, s - start, d)
        ref = oracle.attention_gqa(q.reshape(1, hq, 1, d), np.ascontiguousarray(kd), np.ascontiguousarray(vd),
                                   None, True)
        assert rel_l2(got, ref) <= 1e-6, start


# ---- an independent full-sequence forward -----------------------------------

def _model(oracle, seed: int, nf4: bool, zero_wo_down: bool = False):
    c = CFG
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    shapes = dict(wq=(qd, c["dim"]), wk=(kvd, c["dim"]), wv=(kvd, c["dim"]), wo=(c["dim"], qd),
                  w_gate=(c["ffn"], c["dim"]), w_up=(c["ffn"], c["dim"]), w_down=(c["dim"], c["ffn"]))
    typed, dense = {}, {}
    s = seed
    for name, (n, k) in shapes.items():
        typed[name], dense[name] = [], []
        for _ in range(c["layers"]):
            s += 1
            w = oracle.normal(s, n * k, 0.0, 0.15)
            if zero_wo_down and name in ("wo", "w_down"):
                w = np.zeros(n * k, np.float32)
            if nf4:
                codes, absmax = oracle.nf4_quantize(w, 32)
                typed[name].append((100, codes, absmax))
                dense[name].append(oracle.nf4_dequant(codes, absmax, n * k, 32).reshape(n, k).astype(np.float64))
            else:
                typed[name].append((0, w))
                dense[name].append(w.reshape(n, k).astype(np.float64))
    emb = oracle.normal(s + 1, c["vocab"] * c["dim"])
    head = oracle.normal(s + 2, c["vocab"] * c["dim"], 0.0, 0.1)
    typed["tok_embed"] = (0, emb)
    typed["lm_head"] = (0, head)
    dense["tok_embed"] = emb.reshape(c["vocab"], c["dim"]).astype(np.float64)
    dense["lm_head"] = head.reshape(c["vocab"], c["dim"]).astype(np.float64)
    for key, base in (("attn_norm", s + 3), ("ffn_norm", s + 13)):
        norms = [1.0 + 0.1 * oracle.normal(base + l, c["dim"]) for l in range(c["layers"])]
        typed[key] = [n.astype(np.float32) for n in norms]
        dense[key] = [n.astype(np.float64) for n in norms]
    out_norm = (1.0 + 0.1 * oracle.normal(s + 30, c["dim"])).astype(np.float32)
    typed["out_norm"] = out_norm
    dense["out_norm"] = out_norm.astype(np.float64)
    cfg = dict(c, nf4_block=32)
    return cfg, typed, dense


def _forward(dense, tokens, kv_f16: bool, mistake: str = ""):
    """Causal forward over the whole sequence at once: logits [T, vocab] and
    final hidden states [T, dim]. float64 throughout, except the K/V values
    rounded to binary16 when the cache stores them so."""
    c = CFG
    nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
    half = hd // 2
    n = len(tokens)

    def rmsnorm(x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + c["eps"]) * w

    pos = np.arange(n, dtype=np.float64)[:, None]
    inv = c["rope_base"] ** (-2.0 * np.arange(half) / hd)
    ang = pos * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(x, heads):                                   # x [n, heads*hd]
        x = x.reshape(n, heads, hd).copy()
        if mistake == "interleaved_rope":
            a, b = x[..., 0::2].copy(), x[..., 1::2].copy()
            x[..., 0::2] = a * cos[:, None, :] - b * sin[:, None, :]
            x[..., 1::2] = a * sin[:, None, :] + b * cos[:, None, :]
        else:
            a, b = x[..., :half].copy(), x[..., half:].copy()
            x[..., :half] = a * cos[:, None, :] - b * sin[:, None, :]
            x[..., half:] = a * sin[:, None, :] + b * cos[:, None, :]
        return x

    x = dense["tok_embed"][np.asarray(tokens)]
    for l in range(c["layers"]):
        xn = rmsnorm(x, dense["attn_norm"][l])
        q = rope(xn @ dense["wq"][l].T, nh)
        k = rope(xn @ dense["wk"][l].T, nkv)
        v = (xn @ dense["wv"][l].T).reshape(n, nkv, hd)
        if kv_f16:
            k = k.astype(np.float16).astype(np.float64)
            v = v.astype(np.float16).astype(np.float64)
        att = np.zeros((n, nh, hd))
        for h in range(nh):
            g = h % nkv if mistake == "gqa_modulo" else h // (nh // nkv)
            sc = q[:, h, :] @ k[:, g, :].T / np.sqrt(hd)  # [query, key]
            lim = 0 if mistake == "causal_short" else 1
            mask = np.arange(n)[None, :] < np.arange(n)[:, None] + lim
            if mistake == "causal_short":
                mask[0, 0] = True                        # keep position 0 defined
            sc = np.where(mask, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            att[:, h, :] = p @ v[:, g, :]
        o = att.reshape(n, nh * hd) @ dense["wo"][l].T
        x = o if mistake == "no_attn_residual" else x + o
        xn = rmsnorm(x, dense["ffn_norm"][l])
        gate, up = xn @ dense["w_gate"][l].T, xn @ dense["w_up"][l].T
        if mistake == "gate_up_swapped":
            gate, up = up, gate
        hb = gate / (1.0 + np.exp(-gate)) * up
        x = x + hb @ dense["w_down"][l].T
    logits = rmsnorm(x, dense["out_norm"]) @ dense["lm_head"].T
    return logits, x


def _incremental(oracle, cfg, typed, tokens, kv_f16: bool):
    model = oracle.TypedLlamaOracle(cfg, typed, kv_f16=kv_f16)
    logits, hidden = [], []
    for p, t in enumerate(tokens):
        _, lg, hs = model.decode(int(t), p, 1)
        logits.append(lg.copy())
        hidden.append(hs.copy())
    return np.array(logits), np.array(hidden)


@pytest.mark.parametrize("nf4", [False, True], ids=["f32", "nf4"])
@pytest.mark.parametrize("kv_f16", [False, True], ids=["kv32", "kv16"])
def test_decode_step_equals_full_sequence_forward(oracle, nf4, kv_f16):
    cfg, typed, dense = _model(oracle, 500 + 10 * nf4, nf4)
    tokens = oracle.uniform_int(77, CFG["vocab"], T)
    got_logits, got_hidden = _incremental(oracle, cfg, typed, tokens, kv_f16)
    ref_logits, ref_hidden = _forward(dense, tokens, kv_f16)
    for p in range(T):
        assert rel_l2(got_logits[p], ref_logits[p]) <= 1e-5, p
        assert rel_l2(got_hidden[p], ref_hidden[p]) <= 1e-5, p


@pytest.mark.parametrize("mistake", ["no_attn_residual", "interleaved_rope", "gqa_modulo", "causal_short",
                                     "gate_up_swapped"])
def test_planted_composition_mistakes_are_caught(oracle, mistake):
    """Each mistake in the forward moves some position's logits by far more
    than the tolerance the oracle is held to above."""
    cfg, typed, dense = _model(oracle, 500, False)
    tokens = oracle.uniform_int(77, CFG["vocab"], T)
    got_logits, _ = _incremental(oracle, cfg, typed, tokens, False)
    bad_logits, _ = _forward(dense, tokens, False, mistake)
    worst = max(rel_l2(got_logits[p], bad_logits[p]) for p in range(T))
    assert worst > 1e-2, (mistake, worst)


def test_zero_wo_and_down_leave_the_embedding_row(oracle):
    """With Wo = W_down = 0 each layer adds nothing to x, so the final hidden
    state is the embedding row and logits = lm_head . (rmsnorm(row) * out_norm),
    at every position and whatever the cache holds."""
    cfg, typed, dense = _model(oracle, 900, False, zero_wo_down=True)
    tokens = oracle.uniform_int(91, CFG["vocab"], 6)
    got_logits, got_hidden = _incremental(oracle, cfg, typed, tokens, True)
    for p, t in enumerate(tokens):
        row = dense["tok_embed"][t]
        norm = row / np.sqrt(np.mean(row * row) + CFG["eps"]) * dense["out_norm"]
        assert np.array_equal(got_hidden[p], row.astype(np.float32)), p
        assert rel_l2(got_logits[p], dense["lm_head"] @ norm) <= 1e-6, p


def test_position_zero_attention_is_the_value_row(oracle):
    """At position 0 the softmax has one key, so each query head's attention
    output is its KV head's value row (Wv x') and the first layer's residual
    adds Wo . (v repeated per group): checked through a one-layer model."""
    cfg, typed, dense = _model(oracle, 1300, False)
    cfg1 = dict(cfg, layers=1)
    typed1 = {k: (v[:1] if isinstance(v, list) else v) for k, v in typed.items()}
    dense1 = {k: (v[:1] if isinstance(v, list) else v) for k, v in dense.items()}
    tok = 7
    model = oracle.TypedLlamaOracle(cfg1, typed1, kv_f16=False)
    _, _, hidden = model.decode(tok, 0, 1)
    c = CFG
    x = dense1["tok_embed"][tok]
    xn = x / np.sqrt(np.mean(x * x) + c["eps"]) * dense1["attn_norm"][0]
    v = (dense1["wv"][0] @ xn).reshape(c["n_kv_heads"], c["head_dim"])
    att = np.repeat(v, c["n_heads"] // c["n_kv_heads"], axis=0).reshape(-1)
    x = x + dense1["wo"][0] @ att
    xn = x / np.sqrt(np.mean(x * x) + c["eps"]) * dense1["ffn_norm"][0]
    g, u = dense1["w_gate"][0] @ xn, dense1["w_up"][0] @ xn
    x = x + dense1["w_down"][0] @ (g / (1 + np.exp(-g)) * u)
    assert rel_l2(hidden, x) <= 1e-6
