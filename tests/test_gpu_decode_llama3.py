"""The decode step at BASELINE configs[4] width: Llama-3-8B shapes (dim 4096,
FFN 14336, 32/8 heads of 128, vocab 128256, NF4 block 64, fp16 LM head).

Two layers against the oracle (oracle.LlamaOracle, GgufDecodePass.java:297-420
restated) with the fp16 KV caches of both prefilled identically and sequences
at different positions up to context 2048, so the split-K attention runs with
many splits, per-sequence lengths and the merge; then all 32 layers at
context 2048 through property checks (finite logits, graph replay = eager,
per-group byte accounting = the algorithmic bytes of one step).

Weights, embeddings and caches are drawn on the device (torch), uploaded or
quantized there (aljabr_rocm_quantize), and downloaded as the oracle's
inputs: both sides compute from identical values.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _host(weights):
    import torch
    out = {}
    for key, val in weights.items():
        def get(t):
            a = t.cpu().numpy()
            return a.view(np.uint16) if t.dtype == torch.float16 else a
        out[key] = [get(t) for t in val] if isinstance(val, list) else get(val)
    return out


def _prefill(model, seed: int, keep_host: bool = True):
    """Fill both fp16 caches with N(0, 1) values, 64 Mi elements per draw
    (the same seed gives the same caches in any session of this shape);
    returns host copies [layers][max_batch][n_kv][max_seq][head_dim] as
    float16 when keep_host."""
    import torch
    from aljabr_amd import abi
    k_ptr, v_ptr = model.kv_cache_ptrs()
    n = model.kv_cache_elems()
    c = model.cfg
    shape = (c["layers"], model.max_batch, c["n_kv_heads"], model.max_seq, c["head_dim"])
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    host = []
    for ptr in (k_ptr, v_ptr):
        parts = []
        off, chunk = 0, 1 << 26
        while off < n:
            m = min(chunk, n - off)
            t = torch.randn(m, generator=g, device="cuda:0").half()
            torch.cuda.synchronize()
            abi.call("aljabr_rocm_memcpy_d2d", ptr + 2 * off, t.data_ptr(), 2 * m)
            abi.call("aljabr_rocm_synchronize")
            if keep_host:
                parts.append(t.cpu().numpy())
            del t
            off += m
        if keep_host:
            host.append(np.concatenate(parts).reshape(shape))
    return host


def _oracle_for(oracle, cfg, host, kc, vc, b, max_seq, typed=False):
    """LlamaOracle (TypedLlamaOracle when `typed`) of sequence b with its
    caches set from the device caches (position-major fp32
    [layers][max_seq][n_kv * head_dim])."""
    make = oracle.TypedLlamaOracle if typed else oracle.LlamaOracle
    ref = make(dict(cfg, max_seq=max_seq), host)
    L, kvd = cfg["layers"], cfg["n_kv_heads"] * cfg["head_dim"]
    ref.k_cache[:] = kc[:, b].transpose(0, 2, 1, 3).reshape(L * max_seq * kvd).astype(np.float32)
    ref.v_cache[:] = vc[:, b].transpose(0, 2, 1, 3).reshape(L * max_seq * kvd).astype(np.float32)
    return ref


@pytest.fixture(scope="module")
def llama3_two_layers(rocm):
    import torch
    from aljabr_amd.llama import LLAMA3_8B, random_weights
    cfg = dict(LLAMA3_8B, layers=2)
    print("\n[llama3 width] drawing 2-layer weights", flush=True)
    weights = random_weights(cfg, seed=11)
    host = _host(weights)
    yield cfg, weights, host
    del weights
    torch.cuda.empty_cache()


@pytest.mark.parametrize("batch", [32, 1])
def test_llama3_width_decode_matches_oracle(rocm, dev, oracle, llama3_two_layers, batch):
    """Two decode steps from prefilled caches: B = 32 with positions 100,
    161, ..., 1930 and 2047 (per-sequence lengths, many attention splits,
    the merge), or B = 1 at position 2047 (the fused batch-1 launches); the
    hidden state and logits of every sequence within 1e-3 of the oracle."""
    import torch
    from aljabr_amd.llama import DeviceLlama
    cfg, weights, host = llama3_two_layers
    max_seq = 2112
    model = DeviceLlama(cfg, weights, max_batch=batch, max_seq=max_seq)
    kc, vc = _prefill(model, seed=31 + batch)
    pos = np.array([100 + 61 * b for b in range(batch - 1)] + [2047], np.int32)
    refs = [_oracle_for(oracle, cfg, host, kc, vc, b, max_seq) for b in range(batch)]
    del kc, vc
    cur = oracle.uniform_int(57 + batch, cfg["vocab"], batch).astype(np.int32)
    logits = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    hid = torch.empty(batch * cfg["dim"], dtype=torch.float32, device="cuda:0")
    for step in range(2):
        print(f"[llama3 width] batch {batch} step {step} positions {pos.min()}..{pos.max()}", flush=True)
        nxt = model.decode(dev.put(cur), dev.put(pos), batch, logits=logits)
        got_tok = dev.get(nxt)
        rocm.call("aljabr_rocm_memcpy_d2d", hid.data_ptr(), model.hidden_ptr(), batch * cfg["dim"] * 4)
        got_logits = dev.get(logits).reshape(batch, -1)
        got_hidden = dev.get(hid).reshape(batch, -1)
        for b in range(batch):
            ref_tok, ref_logits, ref_hidden = refs[b].decode(int(cur[b]), int(pos[b]))
            assert rel_l2(got_hidden[b], ref_hidden) <= TOL, (step, b)
            assert rel_l2(got_logits[b], ref_logits) <= TOL, (step, b)
            assert got_tok[b] == ref_tok or \
                ref_logits[ref_tok] - ref_logits[got_tok[b]] <= 1e-3 * np.abs(ref_logits).max(), (step, b)
            cur[b] = ref_tok
        pos = pos + 1
    model.close()


# GGUF Q4_K_M's mix: Q4_K everywhere but the V and down projections and the
# output head (Q6_K). The Q4_0 mix (Q8_0 V, down and head) runs the Q4_0 /
# Q8_0 matrix-core GEMMs: stacked Q/K and gate/up (with the SwiGLU tail), the
# 7-slice down projection with the residual tail.
MIXES = {
    "q4_k_m": dict(tok_embed=12, wq=12, wk=12, wv=14, wo=12, w_gate=12, w_up=12, w_down=14, lm_head=14),
    "q4_0": dict(tok_embed=2, wq=2, wk=2, wv=8, wo=2, w_gate=2, w_up=2, w_down=8, lm_head=8),
}


@pytest.fixture(scope="module", params=sorted(MIXES))
def llama3_q4_k_m(rocm, oracle, request):
    """Two Llama-3-8B-width layers of random GGUF blocks (the GGUF test
    models' scales) in one of the mixes, as oracle weights and as device
    tensors."""
    import torch
    import gguf_writer as gw
    from aljabr_amd.llama import LLAMA3_8B
    cfg = dict(LLAMA3_8B, layers=2, max_seq=2112)
    print(f"\n[llama3 width {request.param}] drawing 2-layer weights", flush=True)
    _, _, host = gw.llama_model(oracle, cfg, MIXES[request.param], seed=9)

    def put(arr):
        return torch.from_numpy(np.ascontiguousarray(arr)).to("cuda:0")

    dev_w = {"tok_embed": (host["tok_embed"][0], put(host["tok_embed"][1])),
             "lm_head": (host["lm_head"][0], put(host["lm_head"][1])),
             "out_norm": put(host["out_norm"]),
             "attn_norm": [put(a) for a in host["attn_norm"]], "ffn_norm": [put(a) for a in host["ffn_norm"]]}
    for key in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
        dev_w[key] = [(t, put(a)) for t, a in host[key]]
    torch.cuda.synchronize()
    yield cfg, dev_w, host
    del dev_w
    torch.cuda.empty_cache()


def test_llama3_width_q4_k_m_decode_matches_oracle(rocm, dev, oracle, llama3_q4_k_m):
    """A GGUF mix at B = 32 (the quantized matrix-core GEMMs with their fused
    tails; Q4_K_M's two formats per Q/K/V launch) from prefilled caches at
    positions 100, 161, ..., 1930 and 2047, two steps: hidden state and
    logits of every sequence within 1e-3 of the typed oracle."""
    import torch
    from aljabr_amd.llama import DeviceLlama
    cfg, dev_w, host = llama3_q4_k_m
    batch, max_seq = 32, cfg["max_seq"]
    model = DeviceLlama.typed(cfg, dev_w, max_batch=batch, max_seq=max_seq)
    kc, vc = _prefill(model, seed=77)
    pos = np.array([100 + 61 * b for b in range(batch - 1)] + [2047], np.int32)
    refs = [_oracle_for(oracle, cfg, host, kc, vc, b, max_seq, typed=True) for b in range(batch)]
    del kc, vc
    cur = oracle.uniform_int(91, cfg["vocab"], batch).astype(np.int32)
    logits = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    hid = torch.empty(batch * cfg["dim"], dtype=torch.float32, device="cuda:0")
    for step in range(2):
        print(f"[llama3 width gguf] step {step} positions {pos.min()}..{pos.max()}", flush=True)
        nxt = model.decode(dev.put(cur), dev.put(pos), batch, logits=logits)
        got_tok = dev.get(nxt)
        rocm.call("aljabr_rocm_memcpy_d2d", hid.data_ptr(), model.hidden_ptr(), batch * cfg["dim"] * 4)
        got_logits = dev.get(logits).reshape(batch, -1)
        got_hidden = dev.get(hid).reshape(batch, -1)
        for b in range(batch):
            ref_tok, ref_logits, ref_hidden = refs[b].decode(int(cur[b]), int(pos[b]))
            assert np.isfinite(got_logits[b]).all(), (step, b)
            assert rel_l2(got_hidden[b], ref_hidden) <= TOL, (step, b)
            assert rel_l2(got_logits[b], ref_logits) <= TOL, (step, b)
            assert got_tok[b] == ref_tok or \
                ref_logits[ref_tok] - ref_logits[got_tok[b]] <= 1e-3 * np.abs(ref_logits).max(), (step, b)
            cur[b] = ref_tok
        pos = pos + 1
    model.close()


def test_llama3_width_gguf_graph_replays_match_eager(rocm, dev, llama3_q4_k_m):
    """A GGUF mix at B = 32 replayed from a captured step graph against eager
    steps of a twin session (the same device weights, caches filled with the
    same values): tokens and logits bit-identical at every step. Inside the
    graph: the quantized matrix-core GEMMs, their slice tails, and for Q4_K_M
    the fp16 activation image the residual tails write for the Q4_K gate/up
    GEMM."""
    import torch
    from aljabr_amd.llama import DeviceLlama
    cfg, dev_w, _ = llama3_q4_k_m
    batch, max_seq = 32, cfg["max_seq"]
    eager = DeviceLlama.typed(cfg, dev_w, max_batch=batch, max_seq=max_seq)
    graph = DeviceLlama.typed(cfg, dev_w, max_batch=batch, max_seq=max_seq)
    for m in (eager, graph):
        _prefill(m, 78, keep_host=False)
    pos = np.array([100 + 61 * b for b in range(batch - 1)] + [2040], np.int32)
    cur = np.random.default_rng(5).integers(0, cfg["vocab"], batch).astype(np.int32)
    le = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    lg = torch.empty_like(le)
    for step in range(4):
        print(f"[llama3 width gguf graph] step {step} positions {pos.min()}..{pos.max()}", flush=True)
        te = dev.get(eager.decode(dev.put(cur), dev.put(pos), batch, logits=le))
        tg = dev.get(graph.decode_graph(dev.put(cur), dev.put(pos), batch, logits=lg))
        got_e, got_g = dev.get(le), dev.get(lg)
        assert np.all(np.isfinite(got_e)), step
        assert np.array_equal(te, tg) and np.array_equal(got_e, got_g), step
        cur = te.astype(np.int32)
        pos = pos + 1
    eager.close()
    graph.close()


@pytest.fixture(scope="module")
def llama3_full(rocm):
    import torch
    from aljabr_amd.llama import LLAMA3_8B, random_weights
    print("\n[llama3 32 layers] drawing weights", flush=True)
    weights = random_weights(LLAMA3_8B, seed=1)
    yield LLAMA3_8B, weights
    del weights
    torch.cuda.empty_cache()


# Algorithmic bytes of one step at context 2048 (every NF4 projection of the
# 32 layers once, the fp16 LM head once, the visible fp16 K and V rows).
NF4_BYTES = 3_925_868_544
HEAD_BYTES = 1_050_673_152
KV_BYTES_PER_SEQ = 268_435_456


@pytest.mark.parametrize("batch", [1, 32])
def test_llama3_full_depth_properties(rocm, dev, llama3_full, batch):
    import torch
    from aljabr_amd.llama import DeviceLlama
    cfg, weights = llama3_full
    max_seq = 2056
    eager = DeviceLlama(cfg, weights, max_batch=batch, max_seq=max_seq)
    graph = DeviceLlama(cfg, weights, max_batch=batch, max_seq=max_seq)
    for m in (eager, graph):
        _prefill(m, 5, keep_host=False)         # the same values in both sessions
    rng = np.random.default_rng(batch)
    cur = rng.integers(0, cfg["vocab"], batch).astype(np.int32)
    le = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    lg = torch.empty_like(le)
    for step in range(3):
        pos = np.full(batch, 2047 + step, np.int32)
        print(f"[llama3 32 layers] batch {batch} step {step}", flush=True)
        te = dev.get(eager.decode(dev.put(cur), dev.put(pos), batch, logits=le))
        tg = dev.get(graph.decode_graph(dev.put(cur), dev.put(pos), batch, logits=lg))
        got_e, got_g = dev.get(le), dev.get(lg)
        assert np.all(np.isfinite(got_e)) and np.all(np.isfinite(got_g)), step
        # Every launch of the step sums in a fixed order (the batched GEMMs
        # add their K slices in slice order, no float atomics), so the replay
        # is bit-identical to the eager step at any batch.
        assert np.array_equal(te, tg) and rel_l2(got_g, got_e) == 0.0, step
        cur = te.astype(np.int32)
    # One profiled step at context 2048: the groups account the step's bytes.
    pos = np.full(batch, 2047, np.int32)
    _, groups = eager.decode_profile(dev.put(cur), dev.put(pos), batch)
    total = sum(g["bytes"] for g in groups)
    expected = NF4_BYTES + HEAD_BYTES + KV_BYTES_PER_SEQ * batch
    # The groups also count the activation rows they read and write (the
    # token rows in and out of every launch, the output clearing of the
    # batched GEMMs), which the weight + KV figure leaves out: about 7% of
    # the step at B = 32, under 0.1% at B = 1.
    assert expected <= total <= expected * (1.08 if batch > 1 else 1.01), (total, expected)
    assert all(g["us"] > 0 for g in groups)
    eager.close()
    graph.close()
