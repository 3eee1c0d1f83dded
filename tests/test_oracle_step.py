"""Pins of the registered whole-step oracle orc_step_decode (CPU only).

The oracle restates the Metal decode step (MTLC/aljabr_metal_matvec_api.m:
3574-4083). It is pinned three ways: with every per-layer feature off and the
SiLU activation it equals orc_llama_decode_typed (itself pinned by the
reference's attention KATs and a full-sequence forward); with every feature on
it equals the independent full-sequence float64 forward in step_models.py at
every position; and mistakes planted in that forward (post norm after the
residual, a window one key too wide, RoPE divisors multiplied, K-as-V taken
after RoPE, a missing unit V norm, the wrong cache owner, the output scale on
the branch only, no softcap) each move the result far past the tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
import step_models as sm

EPS = 1e-6
T = 14


def _run(orc, model, inputs, window):
    o = orc.StepOracle(model)
    out = [o.decode(p, window, EPS, x_in=inputs[p]) for p in range(len(inputs))]
    assert all(rc >= 0 for rc, _, _ in out), [rc for rc, _, _ in out]
    return np.array([lg for _, _, lg in out]), np.array([x for _, x, _ in out]), [rc for rc, _, _ in out]


def test_features_off_equals_llama_oracle(oracle):
    model = sm.llama_like(oracle)
    tokens = oracle.uniform_int(5, sm.VOCAB, 10)
    typed = dict(tok_embed=model["embd"], lm_head=model["out_w"], out_norm=model["out_norm"],
                 attn_norm=list(model["norm"][3].reshape(-1, sm.DIM)),
                 ffn_norm=list(model["norm"][1].reshape(-1, sm.DIM)))
    for key, mk in (("wq", "wq"), ("wk", "wk"), ("wv", "wv"), ("wo", "wo"), ("w_gate", "gate"),
                    ("w_up", "up"), ("w_down", "down")):
        typed[key] = [c[mk] for c in model["layers"]]
    cfg = dict(layers=2, dim=sm.DIM, ffn=sm.FFN, n_heads=sm.NH, n_kv_heads=sm.NKV, head_dim=sm.HD,
               vocab=sm.VOCAB, max_seq=16, rope_base=10000.0, eps=EPS)
    ref = oracle.TypedLlamaOracle(cfg, typed, kv_f16=False)
    step = oracle.StepOracle(model)
    for p, t in enumerate(tokens):
        best_ref, lg_ref, x_ref = ref.decode(int(t), p)
        best, x, lg = step.decode(p, 0, EPS, token=int(t))
        assert rel_l2(lg, lg_ref) <= 1e-5 and rel_l2(x, x_ref) <= 1e-5, p
        assert best == best_ref, p


@pytest.mark.parametrize("use_tokens", [False, True], ids=["x_in", "token"])
def test_every_feature_equals_full_sequence_forward(oracle, use_tokens):
    model, window = sm.gemma_like(oracle)
    tokens = oracle.uniform_int(17, sm.VOCAB, T)
    inputs = sm.token_inputs(model, tokens)
    o = oracle.StepOracle(model)
    got_lg, got_x = [], []
    for p in range(T):
        if use_tokens:
            rc, x, lg = o.decode(p, window, EPS, token=int(tokens[p]))
        else:
            rc, x, lg = o.decode(p, window, EPS, x_in=inputs[p])
        assert rc == int(np.argmax(lg)), p
        got_lg.append(lg)
        got_x.append(x)
    ref_lg, ref_x = sm.forward(model, inputs, window, EPS)
    for p in range(T):
        assert rel_l2(got_lg[p], ref_lg[p]) <= 1e-5, p
        assert rel_l2(got_x[p], ref_x[p]) <= 1e-5, p
    assert np.abs(np.array(got_lg)).max() < model["cap"]


@pytest.mark.parametrize("mistake", ["post_norm_after_residual", "window_off_by_one", "freq_factor_multiplied",
                                     "kv_as_v_after_rope", "unit_v_norm_missing", "shared_kv_wrong_owner",
                                     "out_scale_on_branch", "softcap_missing"])
def test_planted_mistakes_are_caught(oracle, mistake):
    model, window = sm.gemma_like(oracle)
    inputs = sm.token_inputs(model, oracle.uniform_int(17, sm.VOCAB, T))
    got_lg, got_x, _ = _run(oracle, model, inputs, window)
    bad_lg, bad_x = sm.forward(model, inputs, window, EPS, mistake)
    worst = max(max(rel_l2(got_lg[p], bad_lg[p]), rel_l2(got_x[p], bad_x[p])) for p in range(T))
    assert worst > 1e-2, (mistake, worst)


def test_wide_window_equals_no_window(oracle):
    """A sliding window at least as long as the sequence hides nothing."""
    model, _ = sm.gemma_like(oracle)
    inputs = sm.token_inputs(model, oracle.uniform_int(3, sm.VOCAB, 8))
    a, xa, _ = _run(oracle, model, inputs, 8)
    b, xb, _ = _run(oracle, model, inputs, 0)
    assert np.array_equal(a, b) and np.array_equal(xa, xb)


def test_unit_divisors_equal_no_divisors(oracle):
    model, window = sm.gemma_like(oracle)
    inputs = sm.token_inputs(model, oracle.uniform_int(4, sm.VOCAB, 6))
    a, _, _ = _run(oracle, model, inputs, window)
    for c in model["layers"]:
        if c.get("rope_freqs") is not None:
            c["rope_freqs"] = np.ones(sm.HD // 2, np.float32)
    b, _, _ = _run(oracle, model, inputs, window)
    for c in model["layers"]:
        c.pop("rope_freqs", None)
    c_, _, _ = _run(oracle, model, inputs, window)
    assert np.array_equal(b, c_)
    assert rel_l2(a, b) > 1e-3          # the divisors do change the result


def test_missing_kv_owner_is_rejected(oracle):
    """A layer whose cache chain ends at a layer without K is -4, and the
    required norms missing is -3, as the reference returns."""
    model, window = sm.gemma_like(oracle)
    model["layers"][2]["kv_layer"] = 2                # itself, and it has no K projection
    rc, _, _ = oracle.StepOracle(model).decode(0, window, EPS, x_in=np.ones(sm.DIM, np.float32))
    assert rc == -4
    model, window = sm.gemma_like(oracle)
    model["norm"][1] = None
    rc, _, _ = oracle.StepOracle(model).decode(0, window, EPS, x_in=np.ones(sm.DIM, np.float32))
    assert rc == -3
