"""The prefill (FA4) attention oracle, pinned without a GPU: the reference's
uniform-attention fixture, the decode/dense attention oracle (itself pinned
by the reference's known-answer tests) where the two semantics coincide,
prefix invariance of the causal limit for T > S, and closed forms of the soft
cap and the window."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2


def _qkv(oracle, b, t, s, h, hkv, d, seed):
    q = oracle.normal(seed, b * t * h * d).reshape(b, t, h, d)
    k = oracle.normal(seed + 1, b * s * hkv * d).reshape(b, s, hkv, d)
    v = oracle.normal(seed + 2, b * s * hkv * d).reshape(b, s, hkv, d)
    return q, k, v


def test_reference_uniform_attention_fixture(oracle):
    """backend/cpu/.../FlashAttentionCpuTest.java:12-35: zero queries and keys,
    V[i] = (2i, 2i+1) over 65 keys -> every row is the mean of V."""
    q = np.zeros((1, 65, 1, 2), np.float32)
    k = np.zeros((1, 65, 1, 2), np.float32)
    v = np.arange(130, dtype=np.float32).reshape(1, 65, 1, 2)
    out = oracle.fa4_attention(q, k, v, scale=1.0 / np.sqrt(2.0), causal=False)
    expected = np.broadcast_to(v.reshape(65, 2).astype(np.float64).mean(axis=0), (65, 2))
    np.testing.assert_allclose(out.reshape(65, 2), expected, atol=1e-4)


@pytest.mark.parametrize("t,s", [(1, 40), (16, 16), (7, 33), (33, 33)])
@pytest.mark.parametrize("causal", [False, True])
def test_equals_dense_attention_oracle(oracle, t, s, causal):
    """For S >= T both use the bottom-right causal limit S - T + t + 1
    (CPU/CpuBackend.java:1690-1700 vs aljabr_metal_fa4.m:111-115); the dense
    oracle takes [B,H,S,D] layouts and the 1/sqrt(D) scale."""
    b, h, hkv, d = 2, 6, 2, 16
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=5 + t + s)
    out = oracle.fa4_attention(q, k, v, scale=1.0 / np.sqrt(d), causal=causal)
    qd = np.ascontiguousarray(q.transpose(0, 2, 1, 3))
    kd = np.ascontiguousarray(k.transpose(0, 2, 1, 3))
    vd = np.ascontiguousarray(v.transpose(0, 2, 1, 3))
    ref = oracle.attention_gqa(qd, kd, vd, causal=causal)
    assert rel_l2(out, np.ascontiguousarray(ref.transpose(0, 2, 1, 3))) <= 1e-6


def test_causal_limit_when_queries_outnumber_keys(oracle):
    """T > S: row t sees min(t + 1, S) keys (the offset max(S - T, 0) is 0), so
    each row equals a one-row problem over that prefix of the keys."""
    b, t, s, h, hkv, d = 1, 12, 5, 4, 2, 8
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=41)
    out = oracle.fa4_attention(q, k, v, scale=0.3, causal=True)
    for row in range(t):
        n = min(row + 1, s)
        one = oracle.fa4_attention(q[:, row:row + 1], k[:, :n], v[:, :n], scale=0.3, causal=False)
        assert rel_l2(out[:, row], one[:, 0]) <= 1e-7, row


def test_uniform_keys_average_the_visible_values(oracle):
    """Identical keys give every visible key the same weight: row t is the
    mean of V over its causal prefix, whatever Q holds."""
    b, t, s, h, hkv, d = 1, 9, 14, 2, 1, 8
    q, _, v = _qkv(oracle, b, t, s, h, hkv, d, seed=3)
    k = np.broadcast_to(oracle.normal(9, d).reshape(1, 1, 1, d), (b, s, hkv, d)).copy()
    out = oracle.fa4_attention(q, k, v, scale=0.5, causal=True)
    for row in range(t):
        n = s - t + row + 1
        mean = v[0, :n, 0].astype(np.float64).mean(axis=0)
        for head in range(h):
            np.testing.assert_allclose(out[0, row, head], mean, rtol=1e-5, atol=1e-6)


def test_soft_cap_limits(oracle):
    """A huge cap leaves the scores as they are; a tiny cap squeezes them to
    ~0, which averages the visible values."""
    b, t, s, h, hkv, d = 1, 6, 10, 2, 2, 8
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=17)
    plain = oracle.fa4_attention(q, k, v, scale=0.4, causal=True)
    wide = oracle.fa4_attention(q, k, v, scale=0.4, causal=True, soft_cap=1e6)
    assert rel_l2(wide, plain) <= 1e-6
    tight = oracle.fa4_attention(q, k, v, scale=0.4, causal=True, soft_cap=1e-6)
    for row in range(t):
        n = s - t + row + 1
        np.testing.assert_allclose(tight[0, row], v[0, :n].astype(np.float64).mean(axis=0), rtol=1e-4, atol=1e-5)
    assert rel_l2(tight, plain) > 1e-2


def test_window(oracle):
    """window = 1 keeps only the last visible key (out = that V row); a window
    of at least S changes nothing; window w equals the plain problem over the
    w keys below the limit."""
    b, t, s, h, hkv, d = 1, 7, 11, 4, 2, 8
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=23)
    one = oracle.fa4_attention(q, k, v, scale=0.4, causal=True, window=1)
    for row in range(t):
        last = s - t + row
        for head in range(h):
            np.testing.assert_allclose(one[0, row, head], v[0, last, head // 2], rtol=1e-6)
    big = oracle.fa4_attention(q, k, v, scale=0.4, causal=True, window=s)
    plain = oracle.fa4_attention(q, k, v, scale=0.4, causal=True)
    assert rel_l2(big, plain) == 0.0
    w = 3
    win = oracle.fa4_attention(q, k, v, scale=0.4, causal=True, window=w)
    for row in range(t):
        hi = s - t + row + 1
        lo = max(hi - w, 0)
        ref = oracle.fa4_attention(q[:, row:row + 1], k[:, lo:hi], v[:, lo:hi], scale=0.4, causal=False)
        assert rel_l2(win[:, row], ref[:, 0]) <= 1e-7


def test_rejects_bad_head_grouping(oracle):
    q = np.zeros((1, 2, 3, 4), np.float32)
    k = np.zeros((1, 2, 2, 4), np.float32)
    with pytest.raises(ValueError):
        oracle.fa4_attention(q, k, k, scale=1.0)
