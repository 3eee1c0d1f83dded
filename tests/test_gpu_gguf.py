"""GPU parity of the GGUF bridge: Llama-family GGUF files written by
tests/gguf_writer.py are loaded by aljabr_rocm_llama_create_gguf and decoded on
the device; every step is compared with the oracle's typed decode
(GgufDecodePass over per-tensor GGUF types, restated) on the same weights:
hidden state and logits within 1e-3 relative L2, greedy tokens equal up to
near-ties. Also: a session built from device buffers (create_typed) equals
the file-loaded one, graph replays equal eager steps, and files the step
cannot decode faithfully are refused."""
from __future__ import annotations

import numpy as np
import pytest

import gguf_writer as gw
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, dim=512, ffn=1536, n_heads=8, n_kv_heads=2, head_dim=64, vocab=1024, max_seq=16,
           rope_base=500000.0, eps=1e-5)
CFG_BIG = dict(layers=2, dim=2048, ffn=4096, n_heads=16, n_kv_heads=4, head_dim=128, vocab=512, max_seq=16,
               rope_base=500000.0, eps=1e-5)
# Llama-3-8B attention width (32/8 heads of 128 over 4096): the batch-1 Q/K/V
# launch of two row formats at the shipped tile shape (6 Q4_K rows per wave,
# 8 Q6_K rows per wave, 246 workgroups).
CFG_WIDE = dict(layers=2, dim=4096, ffn=2048, n_heads=32, n_kv_heads=8, head_dim=128, vocab=512, max_seq=16,
                rope_base=500000.0, eps=1e-5)
# Q4_K_M-like mix; every supported type; tied LM head; K % 2048 (batch-1 rows kernels).
MIXES = {
    "q4_k_m": (CFG, dict(tok_embed=gw.Q4_K, wq=gw.Q4_K, wk=gw.Q4_K, wv=gw.Q6_K, wo=gw.Q4_K, w_gate=gw.Q4_K,
                         w_up=gw.Q4_K, w_down=gw.Q6_K, lm_head=gw.Q6_K)),
    "all_types": (CFG, dict(tok_embed=gw.Q8_0, wq=gw.Q4_0, wk=gw.Q8_0, wv=gw.F16, wo=gw.F32, w_gate=gw.Q6_K,
                            w_up=gw.Q4_K, w_down=gw.Q8_0, lm_head=gw.F16)),
    "tied_f16": (CFG, dict(tok_embed=gw.F16, wq=gw.Q8_0, wk=gw.Q8_0, wv=gw.Q8_0, wo=gw.Q8_0, w_gate=gw.Q4_0,
                           w_up=gw.Q4_0, w_down=gw.Q4_0, lm_head=None)),
    "rows_k4096_q4_k_m": (CFG_WIDE, dict(tok_embed=gw.Q4_K, wq=gw.Q4_K, wk=gw.Q4_K, wv=gw.Q6_K, wo=gw.Q4_K,
                                         w_gate=gw.Q4_K, w_up=gw.Q4_K, w_down=gw.Q6_K, lm_head=gw.Q6_K)),
    "rows_k2048": (CFG_BIG, dict(tok_embed=gw.Q6_K, wq=gw.Q4_K, wk=gw.Q4_K, wv=gw.Q6_K, wo=gw.Q4_K,
                                 w_gate=gw.Q4_K, w_up=gw.Q4_K, w_down=gw.Q6_K, lm_head=gw.Q6_K)),
    # Batch-1 fused launches per format: one-type Q/K/V (RoPE + append
    # epilogue) in Q8_0 and Q6_K, Q4_0 and Q4_K residual adds, a mixed gate/up.
    "rows_q8": (CFG_BIG, dict(tok_embed=gw.Q8_0, wq=gw.Q8_0, wk=gw.Q8_0, wv=gw.Q8_0, wo=gw.Q4_0, w_gate=gw.Q4_K,
                              w_up=gw.Q4_K, w_down=gw.Q8_0, lm_head=gw.F16)),
    "rows_q6_mixed": (CFG_BIG, dict(tok_embed=gw.F32, wq=gw.Q6_K, wk=gw.Q6_K, wv=gw.Q6_K, wo=gw.Q4_K,
                                    w_gate=gw.Q4_K, w_up=gw.Q6_K, w_down=gw.Q4_0, lm_head=None)),
}


def _write(oracle, tmp_path, name, seed=2):
    cfg, types = MIXES[name]
    meta, tensors, weights = gw.llama_model(oracle, cfg, types, seed=seed)
    path = str(tmp_path / f"{name}.gguf")
    gw.write_gguf(path, meta, tensors)
    return cfg, path, weights


def _run_against_oracle(dev, oracle, model, cfg, weights, batch, steps=5, graph=False):
    import torch
    refs = [oracle.TypedLlamaOracle(cfg, weights) for _ in range(batch)]
    first = (np.array([5, 17, 901], np.int32) % cfg["vocab"])[:batch]
    start = np.array([0, 1, 3], np.int32)[:batch]
    logits = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    cur = first.copy()
    for step in range(steps):
        pos = np.maximum(0, step - start).astype(np.int32)
        cur = np.where(pos == 0, first, cur).astype(np.int32)
        run = model.decode_graph if graph else model.decode
        nxt = run(dev.put(cur), dev.put(pos), batch, logits=logits)
        got_tok = dev.get(nxt)
        got_logits = dev.get(logits).reshape(batch, -1)
        for b in range(batch):
            ref_tok, ref_logits, _ = refs[b].decode(int(cur[b]), int(pos[b]))
            assert np.isfinite(got_logits[b]).all(), (step, b)
            assert rel_l2(got_logits[b], ref_logits) <= 1e-3, (step, b)
            assert got_tok[b] == ref_tok or \
                ref_logits[ref_tok] - ref_logits[got_tok[b]] <= 1e-3 * np.abs(ref_logits).max()
            cur[b] = ref_tok


@pytest.mark.parametrize("name,batch", [("q4_k_m", 1), ("q4_k_m", 3), ("all_types", 1), ("all_types", 2),
                                        ("tied_f16", 2), ("rows_k2048", 1), ("rows_k2048", 3), ("rows_k4096_q4_k_m", 1),
                                        ("rows_k4096_q4_k_m", 2), ("rows_q8", 1),
                                        ("rows_q6_mixed", 1), ("rows_q6_mixed", 2)])
def test_gguf_file_decode_matches_oracle(rocm, dev, oracle, tmp_path, name, batch):
    from aljabr_amd.llama import DeviceLlama
    cfg, path, weights = _write(oracle, tmp_path, name)
    model = DeviceLlama.from_gguf(path, max_batch=batch, max_seq=cfg["max_seq"])
    for key in ("layers", "dim", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab"):
        assert model.cfg[key] == cfg[key], key
    _run_against_oracle(dev, oracle, model, cfg, weights, batch)
    model.close()


def test_typed_session_and_graph_replays(rocm, dev, oracle, tmp_path):
    """The same model from device buffers (create_typed), replayed from a
    captured graph, matches the oracle at every step."""
    import torch
    from aljabr_amd.llama import DeviceLlama
    cfg, _, weights = _write(oracle, tmp_path, "q4_k_m", seed=4)

    def put(arr):
        return torch.from_numpy(np.ascontiguousarray(arr)).to("cuda:0")

    w = {"tok_embed": (weights["tok_embed"][0], put(weights["tok_embed"][1])),
         "lm_head": (weights["lm_head"][0], put(weights["lm_head"][1])),
         "out_norm": put(weights["out_norm"]),
         "attn_norm": [put(a) for a in weights["attn_norm"]], "ffn_norm": [put(a) for a in weights["ffn_norm"]]}
    for key in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
        w[key] = [(t, put(a)) for t, a in weights[key]]
    torch.cuda.synchronize()
    model = DeviceLlama.typed(cfg, w, max_batch=2, max_seq=cfg["max_seq"])
    _run_against_oracle(dev, oracle, model, cfg, weights, 2, steps=5, graph=True)
    model.close()


@pytest.mark.parametrize("extra", ["blk.0.attn_q_norm.weight", "rope_freqs.weight"])
def test_gguf_refuses_what_the_step_does_not_apply(rocm, oracle, tmp_path, extra):
    from aljabr_amd import abi
    from aljabr_amd.llama import DeviceLlama
    cfg, types = MIXES["q4_k_m"]
    meta, tensors, _ = gw.llama_model(oracle, cfg, types)
    tensors.append((extra, [cfg["head_dim"]], gw.F32, np.ones(cfg["head_dim"], np.float32).tobytes()))
    path = str(tmp_path / "extra.gguf")
    gw.write_gguf(path, meta, tensors)
    with pytest.raises(abi.RocmError) as e:
        DeviceLlama.from_gguf(path, max_batch=1, max_seq=8)
    assert e.value.status == abi.ERR_UNSUPPORTED


def test_gguf_missing_tensor(rocm, oracle, tmp_path):
    from aljabr_amd import abi
    from aljabr_amd.llama import DeviceLlama
    cfg, types = MIXES["q4_k_m"]
    meta, tensors, _ = gw.llama_model(oracle, cfg, types)
    tensors = [t for t in tensors if t[0] != "blk.1.ffn_up.weight"]
    path = str(tmp_path / "missing.gguf")
    gw.write_gguf(path, meta, tensors)
    with pytest.raises(abi.RocmError) as e:
        DeviceLlama.from_gguf(path, max_batch=1, max_seq=8)
    assert e.value.status == abi.ERR_BAD_ARGUMENT
