"""A captured decode step owns every buffer it reads. The library's stream
scratch grows by freeing the old buffer, so a graph that had captured its
address would read freed memory once a larger step ran eagerly on the same
stream. The session therefore sizes its own partial-sum buffer for every
matrix-core GEMM a step of 2..max_batch tokens launches (output head
included), the attention runs only on the session's split buffer, and the
stream scratch refuses requests while the stream is being captured.

Each case runs on a fresh thread (a fresh library stream, so the scratch it
holds starts at zero): capture a batch-2 step, run an eager step at the
session's largest batch, replay batch 2 against an eager twin session
(bit-identical tokens and logits), and check that the stream never took any
scratch."""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2

pytestmark = pytest.mark.gpu

NF4_CFG = dict(layers=2, dim=1024, ffn=2048, n_heads=8, n_kv_heads=2, head_dim=128, vocab=4096,
               nf4_block=64, rope_base=500000.0, eps=1e-5)
GGUF_CFG = dict(layers=2, dim=512, ffn=1536, n_heads=8, n_kv_heads=2, head_dim=64, vocab=1024, max_seq=16,
                rope_base=500000.0, eps=1e-5)
Q4_K_M = dict(tok_embed=gw.Q4_K, wq=gw.Q4_K, wk=gw.Q4_K, wv=gw.Q6_K, wo=gw.Q4_K, w_gate=gw.Q4_K, w_up=gw.Q4_K,
              w_down=gw.Q6_K, lm_head=gw.Q6_K)
MAX_SEQ = 16


def _nf4_weights(oracle, cfg, nf4_head):
    """Device weights for DeviceLlama.typed: NF4 projections, an fp32
    embedding, and an NF4 or fp16 output head."""
    import torch
    from aljabr_amd import abi
    from aljabr_amd.llama import PROJ, proj_shapes

    def put(a):
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to("cuda:0")

    w = {k: [] for k in PROJ}
    shapes = proj_shapes(cfg)
    for layer in range(cfg["layers"]):
        for i, name in enumerate(PROJ):
            n, k = shapes[name]
            codes, absmax = oracle.nf4_quantize(oracle.normal(50 + 10 * layer + i, n * k, 0.0, 0.02), 64)
            w[name].append((abi.TYPE_NF4, (put(codes), put(absmax))))
    w["attn_norm"] = [put(1.0 + 0.1 * oracle.normal(70 + l, cfg["dim"])) for l in range(cfg["layers"])]
    w["ffn_norm"] = [put(1.0 + 0.1 * oracle.normal(80 + l, cfg["dim"])) for l in range(cfg["layers"])]
    w["out_norm"] = put(1.0 + 0.1 * oracle.normal(90, cfg["dim"]))
    w["tok_embed"] = (abi.TYPE_F32, put(oracle.normal(91, cfg["vocab"] * cfg["dim"])))
    head = oracle.normal(92, cfg["vocab"] * cfg["dim"], 0.0, 0.5)
    if nf4_head:
        codes, absmax = oracle.nf4_quantize(head, 64)
        w["lm_head"] = (abi.TYPE_NF4, (put(codes), put(absmax)))
    else:
        w["lm_head"] = (abi.TYPE_F16, put(head.astype(np.float16).view(np.uint16)))
    torch.cuda.synchronize()
    return w


def _scratch_bytes():
    from aljabr_amd import abi
    n = ctypes.c_size_t(0)
    abi.call("aljabr_rocm_stream_scratch_bytes", ctypes.byref(n))
    return n.value


def _replays_after_a_larger_step(dev, make, cfg, max_batch):
    import torch
    assert _scratch_bytes() == 0
    graph, eager = make(max_batch), make(max_batch)
    vocab = cfg["vocab"]
    lg, le = (torch.empty(max_batch * vocab, dtype=torch.float32, device="cuda:0") for _ in range(2))
    cur = np.array([5, 17], np.int32)
    for step in range(4):
        pos = np.full(2, step, np.int32)
        tg = graph.decode_graph(dev.put(cur), dev.put(pos), 2, logits=lg)
        te = eager.decode(dev.put(cur), dev.put(pos), 2, logits=le)
        torch.cuda.synchronize()
        got_g, got_e = dev.get(tg), dev.get(te)
        assert np.array_equal(got_g, got_e), step
        assert rel_l2(dev.get(lg)[:2 * vocab], dev.get(le)[:2 * vocab]) == 0.0, step
        if step == 0:
            # The largest batch, eagerly, at the last cache row (rows the
            # replays read stay as they were).
            big = (np.arange(max_batch, dtype=np.int32) * 37) % vocab
            graph.decode(dev.put(big), dev.put(np.full(max_batch, MAX_SEQ - 1, np.int32)), max_batch, logits=lg)
            torch.cuda.synchronize()
        cur = got_e.astype(np.int32)
    assert _scratch_bytes() == 0
    graph.close()
    eager.close()


def _on_fresh_thread(fn):
    err = []

    def body():
        try:
            fn()
        except BaseException as e:            # re-raised on the test's thread
            err.append(e)

    t = threading.Thread(target=body)
    t.start()
    t.join(timeout=300)
    assert not t.is_alive(), "worker thread did not finish"
    if err:
        raise err[0]


@pytest.mark.parametrize("head", ["f16", "nf4"])
def test_nf4_graph_replay_after_largest_batch(rocm, dev, oracle, head):
    from aljabr_amd.llama import DeviceLlama
    w = _nf4_weights(oracle, NF4_CFG, head == "nf4")
    # 70 tokens: two GEMM passes (64 + 6) on the register-resident kernel.
    _on_fresh_thread(lambda: _replays_after_a_larger_step(
        dev, lambda b: DeviceLlama.typed(NF4_CFG, w, max_batch=b, max_seq=MAX_SEQ), NF4_CFG, 70))


def test_q4_k_m_graph_replay_after_largest_batch(rocm, dev, oracle, tmp_path):
    from aljabr_amd.llama import DeviceLlama
    meta, tensors, _ = gw.llama_model(oracle, GGUF_CFG, Q4_K_M, seed=3)
    path = str(tmp_path / "q4_k_m.gguf")
    gw.write_gguf(path, meta, tensors)
    # 40 tokens: the K-quant matrix cores in passes of 32 plus the 8 left over.
    _on_fresh_thread(lambda: _replays_after_a_larger_step(
        dev, lambda b: DeviceLlama.from_gguf(path, max_batch=b, max_seq=MAX_SEQ), GGUF_CFG, 40))


def test_stream_scratch_query_rejects_null(rocm):
    from aljabr_amd import abi
    lib = abi.load()
    assert lib.aljabr_rocm_stream_scratch_bytes(None) == abi.ERR_BAD_ARGUMENT
