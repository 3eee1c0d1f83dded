"""GPU parity of the registered whole-step decode and the fused layer entry
points (the Metal ABI's MTLC/aljabr_metal_matvec_api.h:161-282) against the
oracle orc_step_decode (pinned in test_oracle_step.py) on identical inputs.

A small model with every per-layer feature (head norms, unit V norm, post
norms, RoPE divisors, sliding windows, K-as-V, a shared cache, output
scales, softcap) in fp32 weights runs the generic launches; a model at
2048 width with Q4_K/Q6_K/Q8_0 weights runs the fused batch-1 rows launches
(norm prologue, residual and GELU/SiLU epilogues). Weights, norms, inputs and
outputs are passed as host memory in some cases and device memory in
others. Logits must agree within 2e-4 relative L2 and the greedy token must
match wherever the oracle's top two logits are apart.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import rel_l2
import step_models as sm

pytestmark = pytest.mark.gpu
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
EPS = 1e-6
TOL = 2e-4


class Registry:
    """Registers a step_models-style model through the C ABI."""

    def __init__(self, rocm, dev, model, host: bool):
        self.rocm, self.dev, self.host, self.keep = rocm, dev, host, []
        self.lib = rocm.load()
        rocm.call("aljabr_rocm_reset_decode_state")
        dim, layers = model["dim"], model["layers"]
        n = len(layers)
        strides = (ctypes.c_int * n)(*[c["n_kv_heads"] * c["head_dim"] for c in layers])
        rocm.call("aljabr_rocm_init_kv_cache", n, model["max_seq"], strides)
        for slot, arr in enumerate(model["norm"]):
            if arr is not None:
                rocm.call("aljabr_rocm_register_norm_buffer", slot, self.buf(arr), arr.nbytes)
        for l, c in enumerate(layers):
            mats = ("wq", "wk", "wv", "wo", "gate", "up", "down")
            self.register_layer(l, c, dim, [self.buf(c[m][1]) if c.get(m) is not None else None for m in mats])
            if c.get("rope_freqs") is not None:
                rocm.call("aljabr_rocm_register_rope_freqs", l, self.buf(c["rope_freqs"]), c["rope_freqs"].size)
        rocm.call("aljabr_rocm_register_output", self.buf(model["out_norm"]), self.buf(model["out_w"][1]),
                  model["out_w"][0], dim, model["vocab"], model.get("cap", 0.0))
        rocm.call("aljabr_rocm_register_token_embd", self.buf(model["embd"][1]), model["embd"][0], dim,
                  model.get("embd_scale", 1.0))
        rocm.call("aljabr_rocm_set_decode_activation", model["activation"])
        self.dim, self.vocab = dim, model["vocab"]
        self.logits_dev = dev.empty(self.vocab)

    def register_layer(self, l, c, dim, ptrs, wo_n=None):
        """register_decode_layer for layer `l` of config `c` with the weight
        pointers `ptrs` (wq, wk, wv, wo, gate, up, down)."""
        nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        mats = ("wq", "wk", "wv", "wo", "gate", "up", "down")
        types = [c[m][0] if c.get(m) is not None else 0 for m in mats]
        self.rocm.call("aljabr_rocm_register_decode_layer", l, c.get("kv_layer", l), *ptrs, *types, nh * hd,
                       nkv * hd, nkv * hd, nh * hd, wo_n or dim, c["ffn"], nh, nkv, hd, nkv * hd,
                       c.get("freq_base", 10000.0), int(c.get("is_swa", 0)), c.get("out_scale", 1.0),
                       c.get("attn_scale", 0.0),
                       *[int(c.get(f, 0)) for f in ("has_post_attn_norm", "has_post_ffn_norm", "has_q_norm",
                                                    "has_k_norm", "has_unit_v_norm")])

    def buf(self, a):
        a = np.ascontiguousarray(a)
        if self.host:
            self.keep.append(a)
            return a.ctypes.data
        t = self.dev.put(a)
        self.keep.append(t)
        return self.dev.ptr(t)

    def step(self, pos, window, x_in=None, token=-1):
        """(status, logits): host or device input and output as registered."""
        if self.host:
            logits = np.zeros(self.vocab, np.float32)
            out = logits.ctypes.data
        else:
            out = self.dev.ptr(self.logits_dev)
        if token >= 0:
            rc = self.lib.aljabr_rocm_decode_step_token(pos, window, EPS, token, out)
        else:
            xin = np.ascontiguousarray(x_in, np.float32)
            if self.host:
                rc = self.lib.aljabr_rocm_decode_step(pos, window, EPS, xin.ctypes.data, out)
            else:
                xd = self.dev.put(xin)
                rc = self.lib.aljabr_rocm_decode_step(pos, window, EPS, self.dev.ptr(xd), out)
        if rc < 0:
            raise self.rocm.RocmError(rc, "decode_step", self.rocm.last_error())
        return rc, (logits if self.host else self.dev.get(self.logits_dev))


def _check(got_rc, got, ref_rc, ref, where):
    assert rel_l2(got, ref) <= TOL, (where, rel_l2(got, ref))
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 1e-3 * max(1.0, abs(top2[1])):
        assert got_rc == ref_rc, where


@pytest.mark.parametrize("host", [True, False], ids=["host", "device"])
@pytest.mark.parametrize("use_tokens", [False, True], ids=["x_in", "token"])
def test_gemma_like_step_matches_oracle(rocm, dev, oracle, host, use_tokens):
    model, window = sm.gemma_like(oracle)
    tokens = oracle.uniform_int(17, sm.VOCAB, 16)
    inputs = sm.token_inputs(model, tokens)
    reg = Registry(rocm, dev, model, host)
    orc = oracle.StepOracle(model)
    for p in range(16):
        print(f"gemma_like host={host} tokens={use_tokens} pos={p}", flush=True)
        if use_tokens:
            got_rc, got = reg.step(p, window, token=int(tokens[p]))
            ref_rc, _, ref = orc.decode(p, window, EPS, token=int(tokens[p]))
        else:
            got_rc, got = reg.step(p, window, x_in=inputs[p])
            ref_rc, _, ref = orc.decode(p, window, EPS, x_in=inputs[p])
        _check(got_rc, got, ref_rc, ref, p)


def _typed(oracle, t, n, k, seed):
    if t in (Q4_K, Q6_K):
        return t, oracle.random_k_blocks(t, n * k // 256, seed, scale=0.5 / np.sqrt(k) / (200 if t == Q4_K else 1000))
    w = oracle.normal(seed, n * k, 0.0, 0.5 / np.sqrt(k))
    if t in (Q4_0, Q8_0):
        return t, oracle.quantize(t, w)
    if t == F16:
        return t, w.astype(np.float16).view(np.uint16)
    return t, w.astype(np.float32)


def _wide_model(oracle, activation, qkv_types, seed=900, max_seq=96, dim=2048, ffn=4096, nh=16, nkv=4):
    """Two layers at width 2048 (16 query heads, 4 KV heads of 128, FFN
    4096, vocab 1024) unless given: layer 0 takes the types in qkv_types, Q4_K
    wO and gate/up, Q6_K down; layer 1 Q4_K Q/K, Q6_K V (a Q4_K_M mix), Q8_0
    FFN."""
    hd, vocab = 128, 1024
    layers = []
    specs = [(qkv_types, Q4_K, (Q4_K, Q4_K, Q6_K)), ((Q4_K, Q4_K, Q6_K), Q4_K, (Q8_0, Q8_0, Q8_0))]
    for l, (qkv, wo_t, ffn_t) in enumerate(specs):
        s = seed + 20 * l
        layers.append(dict(wq=_typed(oracle, qkv[0], nh * hd, dim, s + 1), wk=_typed(oracle, qkv[1], nkv * hd, dim, s + 2),
                           wv=_typed(oracle, qkv[2], nkv * hd, dim, s + 3), wo=_typed(oracle, wo_t, dim, nh * hd, s + 4),
                           gate=_typed(oracle, ffn_t[0], ffn, dim, s + 5), up=_typed(oracle, ffn_t[1], ffn, dim, s + 6),
                           down=_typed(oracle, ffn_t[2], dim, ffn, s + 7), n_heads=nh, n_kv_heads=nkv, head_dim=hd,
                           ffn=ffn, freq_base=500000.0))
    norm = [None] * 6
    norm[3] = (1.0 + 0.1 * oracle.normal(seed + 50, 2 * dim)).astype(np.float32)
    norm[1] = (1.0 + 0.1 * oracle.normal(seed + 51, 2 * dim)).astype(np.float32)
    return dict(dim=dim, max_seq=max_seq, activation=activation, vocab=vocab, cap=0.0, embd_scale=1.0, layers=layers,
                norm=norm, out_norm=(1.0 + 0.1 * oracle.normal(seed + 52, dim)).astype(np.float32),
                out_w=_typed(oracle, Q6_K, vocab, dim, seed + 53), embd=_typed(oracle, Q6_K, vocab, dim, seed + 54))


# The last case has Llama-3-8B's attention width (32/8 heads of 128 over 4096):
# layer 1's Q4_K Q/K beside its Q6_K V run as one two-format rows launch at
# the decode shape's tiles (6 Q4_K rows per wave, 8 Q6_K rows per wave).
@pytest.mark.parametrize("activation,qkv_types,shape,P",
                         [(1, (Q4_K, Q4_K, Q4_K), (2048, 4096, 16, 4), 70),
                          (2, (Q8_0, Q8_0, Q8_0), (2048, 4096, 16, 4), 70),
                          (1, (Q4_K, Q4_K, Q6_K), (4096, 2048, 32, 8), 20)],
                         ids=["silu_q4k", "gelu_q8", "silu_q4k_m_width4096"])
def test_wide_quantized_step_with_synced_prefix(rocm, dev, oracle, activation, qkv_types, shape, P):
    """The oracle decodes positions 0..P-1; its caches are loaded with
    sync_kv_cache; both then decode P..P+7 from tokens."""
    dim, ffn, nh, nkv = shape
    model = _wide_model(oracle, activation, qkv_types, dim=dim, ffn=ffn, nh=nh, nkv=nkv)
    tokens = oracle.uniform_int(23, model["vocab"], P + 8)
    orc = oracle.StepOracle(model)
    for p in range(P):
        orc.decode(p, 0, EPS, token=int(tokens[p]))
    reg = Registry(rocm, dev, model, host=False)
    for l in range(2):
        stride = nkv * 128
        k = np.ascontiguousarray(orc.k_cache[l][: P * stride])
        v = np.ascontiguousarray(orc.v_cache[l][: P * stride])
        rocm.call("aljabr_rocm_sync_kv_cache", l, P, k.ctypes.data, v.ctypes.data)
    for p in range(P, P + 8):
        print(f"wide act={activation} pos={p}", flush=True)
        got_rc, got = reg.step(p, 0, token=int(tokens[p]))
        ref_rc, _, ref = orc.decode(p, 0, EPS, token=int(tokens[p]))
        _check(got_rc, got, ref_rc, ref, p)


def test_step_errors(rocm, dev, oracle):
    lib = rocm.load()
    rocm.call("aljabr_rocm_reset_decode_state")
    x = np.ones(sm.DIM, np.float32)
    assert lib.aljabr_rocm_decode_step(0, 0, EPS, x.ctypes.data, None) == rocm.ERR_NOT_INITIALIZED
    model, window = sm.gemma_like(oracle)
    reg = Registry(rocm, dev, model, host=True)
    c = model["layers"][0]
    w = reg.buf(c["wq"][1])
    # a cache owner after the layer, as the reference refuses
    assert lib.aljabr_rocm_register_decode_layer(0, 1, w, w, w, w, w, w, w, *([0] * 7), 64, 32, 32, 64, 64, 96,
                                                 4, 2, 16, 32, 10000.0, 0, 1.0, 0.0, 0, 0, 0, 0, 0) \
        == rocm.ERR_BAD_ARGUMENT
    assert lib.aljabr_rocm_decode_step(model["max_seq"], window, EPS, x.ctypes.data, None) == rocm.ERR_BAD_ARGUMENT
    assert lib.aljabr_rocm_decode_step_token(0, window, EPS, sm.VOCAB, None) == rocm.ERR_BAD_ARGUMENT
    assert lib.aljabr_rocm_set_decode_activation(3) == rocm.ERR_BAD_ARGUMENT
    rc, _ = reg.step(0, window, x_in=x)          # the registry still works after the refusals
    assert rc >= 0
    rocm.call("aljabr_rocm_reset_decode_state")


# ---- the per-layer fused calls --------------------------------------------

def _dense(oracle, pair, n, k):
    t, raw = pair
    if t == F32:
        return np.asarray(raw, np.float64).reshape(n, k)
    if t == F16:
        return np.asarray(raw, np.uint16).view(np.float16).astype(np.float64).reshape(n, k)
    return oracle.dequant(t, raw, n * k).astype(np.float64).reshape(n, k)


def _layer_ref(oracle, x, att, L, norms, act, out_scale):
    """x after wO + norms + FFN + residual, float64 from dequantized weights."""
    dim, k, ffn = L["dim"], L["k"], L["ffn"]

    def rms(v, w=None):
        r = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + EPS)
        return r * w if w is not None else r

    xb = att @ _dense(oracle, L["wo"], dim, k).T
    if norms.get("post_attn") is not None:
        xb = rms(xb, norms["post_attn"])
    x1 = x + xb
    h = rms(x1, norms["ffn"])
    g = h @ _dense(oracle, L["gate"], ffn, dim).T
    u = h @ _dense(oracle, L["up"], ffn, dim).T
    hb = oracle.gated_activation(g, u, act).astype(np.float64)
    d = hb @ _dense(oracle, L["down"], dim, ffn).T
    if norms.get("post_ffn") is not None:
        d = rms(d, norms["post_ffn"])
    x2 = x1 + d
    return x2 * out_scale if out_scale > 0 and out_scale != 1.0 else x2


def _adhoc_layer(oracle, dim=512, k=512, ffn=1024, seed=70):
    return dict(dim=dim, k=k, ffn=ffn, wo=_typed(oracle, Q4_K, dim, k, seed), gate=_typed(oracle, Q8_0, ffn, dim, seed + 1),
                up=_typed(oracle, Q8_0, ffn, dim, seed + 2), down=_typed(oracle, Q6_K, dim, ffn, seed + 3))


@pytest.mark.parametrize("post_norms,act", [(False, 1), (True, 2)], ids=["plain_silu", "post_norms_gelu"])
def test_wo_ffn_next_qkv_fused(rocm, dev, oracle, post_norms, act):
    lib = rocm.load()
    rocm.call("aljabr_rocm_reset_decode_state")
    L = _adhoc_layer(oracle)
    dim = L["dim"]
    x = oracle.normal(1, dim)
    att = oracle.normal(2, L["k"])
    norms = {"ffn": (1 + 0.1 * oracle.normal(3, dim)).astype(np.float32)}
    if post_norms:
        norms["post_attn"] = (1 + 0.1 * oracle.normal(4, dim)).astype(np.float32)
        norms["post_ffn"] = (1 + 0.1 * oracle.normal(5, dim)).astype(np.float32)
    next_norm = (1 + 0.1 * oracle.normal(6, dim)).astype(np.float32)
    nq, nk = _typed(oracle, Q4_K, 512, dim, 80), _typed(oracle, Q6_K, 256, dim, 81)
    nv = _typed(oracle, Q4_K, 256, dim, 82)
    out_scale = 0.5 if post_norms else 1.0
    xin = x.copy()
    q, kk, v = (np.zeros(512, np.float32), np.zeros(256, np.float32), np.zeros(256, np.float32))
    keep = [L[m][1] for m in ("wo", "gate", "up", "down")] + [nq[1], nk[1], nv[1]]
    P = lambda a: None if a is None else np.ascontiguousarray(a).ctypes.data
    rc = lib.aljabr_rocm_wo_ffn_next_qkv_fused(
        P(xin), P(att), P(L["wo"][1]), L["wo"][0], L["k"], dim, P(norms.get("post_attn")), int(post_norms),
        P(norms["ffn"]), P(norms.get("post_ffn")), int(post_norms), EPS, out_scale, P(L["gate"][1]), P(L["up"][1]),
        P(L["down"][1]), L["gate"][0], L["up"][0], L["down"][0], L["ffn"], act, 1, P(next_norm), P(q), P(kk), P(v),
        P(nq[1]), P(nk[1]), P(nv[1]), nq[0], nk[0], nv[0], 512, 256, 256)
    rocm.check(rc, "wo_ffn_next_qkv_fused")
    del keep
    ref_x = _layer_ref(oracle, x.astype(np.float64), att.astype(np.float64), L, norms, act, out_scale)
    assert rel_l2(xin, ref_x) <= TOL
    h = ref_x / np.sqrt(np.mean(ref_x * ref_x) + EPS) * next_norm
    for got, pair, n in ((q, nq, 512), (kk, nk, 256), (v, nv, 256)):
        assert rel_l2(got, _dense(oracle, pair, n, dim) @ h) <= TOL


def test_wo_ffn_fused_and_logits_fused(rocm, dev, oracle):
    lib = rocm.load()
    rocm.call("aljabr_rocm_reset_decode_state")
    L = _adhoc_layer(oracle, seed=170)
    dim = L["dim"]
    x = oracle.normal(11, dim)
    att = oracle.normal(12, L["k"])
    norms = {"ffn": (1 + 0.1 * oracle.normal(13, dim)).astype(np.float32)}
    args = lambda xin: (xin.ctypes.data, att.ctypes.data, L["wo"][1].ctypes.data, L["wo"][0], L["k"], dim)
    # device residual and attention input for this one
    xd, ad = dev.put(x), dev.put(att)
    rc = lib.aljabr_rocm_wo_ffn_fused(dev.ptr(xd), dev.ptr(ad), L["wo"][1].ctypes.data, L["wo"][0], L["k"], dim,
                                      None, 0, 0, norms["ffn"].ctypes.data, 0, None, 0, 0, EPS,
                                      L["gate"][1].ctypes.data, L["up"][1].ctypes.data, L["down"][1].ctypes.data,
                                      L["gate"][0], L["up"][0], L["down"][0], L["ffn"], 2)
    rocm.check(rc, "wo_ffn_fused")
    ref_x = _layer_ref(oracle, x.astype(np.float64), att.astype(np.float64), L, norms, 2, 1.0)
    assert rel_l2(dev.get(xd), ref_x) <= TOL
    vocab, cap = 1000, 4.0
    out_norm = (1 + 0.1 * oracle.normal(14, dim)).astype(np.float32)
    out_w = _typed(oracle, Q4_K, vocab, dim, 15)
    logits = np.zeros(vocab, np.float32)
    xin = x.copy()
    rc = lib.aljabr_rocm_wo_ffn_logits_fused(*args(xin), None, 0, norms["ffn"].ctypes.data, None, 0, EPS, 1.5,
                                             L["gate"][1].ctypes.data, L["up"][1].ctypes.data,
                                             L["down"][1].ctypes.data, L["gate"][0], L["up"][0], L["down"][0],
                                             L["ffn"], 1, out_norm.ctypes.data, out_w[1].ctypes.data, out_w[0], dim,
                                             vocab, logits.ctypes.data, cap)
    rocm.check(rc, "wo_ffn_logits_fused")
    ref_x = _layer_ref(oracle, x.astype(np.float64), att.astype(np.float64), L, norms, 1, 1.5)
    assert rel_l2(xin, ref_x) <= TOL
    h = ref_x / np.sqrt(np.mean(ref_x * ref_x) + EPS) * out_norm
    ref_lg = cap * np.tanh((_dense(oracle, out_w, vocab, dim) @ h) / cap)
    assert rel_l2(logits, ref_lg) <= TOL
    lib.aljabr_rocm_wo_ffn_reset_x()


@pytest.mark.parametrize("batch", [1, 5, 32])
def test_wo_ffn_fused_layer_batch(rocm, dev, oracle, batch):
    """The registered layer 0 of the feature model (post norms, output
    scale 1) and layer 1 (output scale 0.75) over `batch` rows."""
    model, _ = sm.gemma_like(oracle)
    reg = Registry(rocm, dev, model, host=True)
    lib = rocm.load()
    dim = sm.DIM
    for layer in (0, 1):
        c = model["layers"][layer]
        x = oracle.normal(40 + batch, batch * dim).reshape(batch, dim)
        att = oracle.normal(41 + batch, batch * sm.NH * sm.HD).reshape(batch, -1)
        xin = np.ascontiguousarray(x.copy())
        rc = lib.aljabr_rocm_wo_ffn_fused_layer_batch(xin.ctypes.data, att.ctypes.data, layer, batch, EPS, 2)
        rocm.check(rc, "wo_ffn_fused_layer_batch")
        norms = {"ffn": model["norm"][1].reshape(-1, dim)[layer]}
        if c.get("has_post_attn_norm"):
            norms["post_attn"] = model["norm"][0].reshape(-1, dim)[layer]
        if c.get("has_post_ffn_norm"):
            norms["post_ffn"] = model["norm"][2].reshape(-1, dim)[layer]
        L = dict(dim=dim, k=sm.NH * sm.HD, ffn=sm.FFN, wo=c["wo"], gate=c["gate"], up=c["up"], down=c["down"])
        ref = _layer_ref(oracle, x.astype(np.float64), att.astype(np.float64), L, norms, 2, c.get("out_scale", 1.0))
        assert rel_l2(xin, ref) <= TOL, layer
    del reg
    rocm.call("aljabr_rocm_reset_decode_state")


def test_reregistered_layer_reads_new_host_weights(rocm, dev, oracle):
    """Host weights are uploaded once per registration: a layer registered
    again from the same host addresses (same sizes and types) after the
    caller rewrote them computes with the new contents, not a stale copy."""
    model, _ = sm.gemma_like(oracle)
    reg = Registry(rocm, dev, model, host=True)
    lib = rocm.load()
    dim, batch = sm.DIM, 3
    c = model["layers"][0]
    mats = ("wq", "wk", "wv", "wo", "gate", "up", "down")
    own = {m: np.array(c[m][1], copy=True) for m in mats if c.get(m) is not None}
    ptrs = [own[m].ctypes.data if m in own else None for m in mats]
    norms = {"ffn": model["norm"][1].reshape(-1, dim)[0]}
    if c.get("has_post_attn_norm"):
        norms["post_attn"] = model["norm"][0].reshape(-1, dim)[0]
    if c.get("has_post_ffn_norm"):
        norms["post_ffn"] = model["norm"][2].reshape(-1, dim)[0]
    x = oracle.normal(61, batch * dim).reshape(batch, dim)
    att = oracle.normal(62, batch * sm.NH * sm.HD).reshape(batch, -1)
    for rnd in range(2):
        if rnd == 1:                              # same buffers, new weights
            for i, m in enumerate(("wo", "gate", "up", "down")):
                assert c[m][0] == F32
                own[m][...] = oracle.normal(63 + i, own[m].size, 0.0, 0.1).reshape(own[m].shape)
        reg.register_layer(0, c, dim, ptrs)
        xin = np.ascontiguousarray(x.copy())
        rocm.check(lib.aljabr_rocm_wo_ffn_fused_layer_batch(xin.ctypes.data, att.ctypes.data, 0, batch, EPS, 2),
                   "wo_ffn_fused_layer_batch")
        L = dict(dim=dim, k=sm.NH * sm.HD, ffn=sm.FFN, **{m: (F32, own[m]) for m in ("wo", "gate", "up", "down")})
        ref = _layer_ref(oracle, x.astype(np.float64), att.astype(np.float64), L, norms, 2, c.get("out_scale", 1.0))
        assert rel_l2(xin, ref) <= TOL, rnd
    del reg
    rocm.call("aljabr_rocm_reset_decode_state")


def test_layer_batch_refuses_a_layer_wider_than_the_model(rocm, dev, oracle):
    """The batch Wo/FFN call works on rows of the model width (layer 0's);
    a layer registered wider is refused before anything runs."""
    model, _ = sm.gemma_like(oracle)
    reg = Registry(rocm, dev, model, host=True)
    lib = rocm.load()
    wide = sm.DIM + 32
    c = dict(n_heads=2, n_kv_heads=1, head_dim=16, ffn=64, kv_layer=1,
             **{m: (F32, None) for m in ("wq", "wk", "wv", "wo", "gate", "up", "down")})
    shapes = dict(wq=(32, wide), wk=(16, wide), wv=(16, wide), wo=(wide, 32), gate=(64, wide), up=(64, wide),
                  down=(wide, 64))
    ptrs = [reg.buf(np.full(shapes[m], 0.01, np.float32)) for m in ("wq", "wk", "wv", "wo", "gate", "up", "down")]
    reg.register_layer(1, c, sm.DIM, ptrs, wo_n=wide)
    x = np.zeros(2 * wide, np.float32)
    att = np.zeros(2 * 32, np.float32)
    assert lib.aljabr_rocm_wo_ffn_fused_layer_batch(x.ctypes.data, att.ctypes.data, 1, 2, EPS, 2) \
        == rocm.ERR_BAD_ARGUMENT
    assert "width" in rocm.last_error()
    del reg
    rocm.call("aljabr_rocm_reset_decode_state")
