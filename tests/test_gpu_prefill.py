"""GPU parity of the prefill (FA4) attention entry points against the oracle
on identical seeded inputs: relative L2 <= 1e-3 per case (fp32 outputs).
Covers the matrix-core kernel (D = 64 and 128, one and two row tiles per
wave: causal T = S, chunked prefill S > T, T > S, partial tiles and blocks,
MHA / GQA / G = 8, batches, soft cap, windows, non-causal) and the generic
kernel (other D, unaligned pointers, the reference's uniform-attention
fixture). At the Llama-3-8B prefill size the
rows are checked one by one on a sample against one-row oracle problems."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _qkv(oracle, b, t, s, h, hkv, d, seed):
    q = oracle.normal(seed, b * t * h * d).reshape(b, t, h, d)
    k = oracle.normal(seed + 1, b * s * hkv * d).reshape(b, s, hkv, d)
    v = oracle.normal(seed + 2, b * s * hkv * d).reshape(b, s, hkv, d)
    return q, k, v


def _run(rocm, dev, q, k, v, scale, causal, soft_cap=0.0, window=0):
    b, t, h, d = q.shape
    s, hkv = k.shape[1], k.shape[2]
    qd, kd, vd = dev.put(q), dev.put(k), dev.put(v)
    out = dev.empty(q.size)
    if window:
        rocm.call("aljabr_rocm_fa4_attention_windowed", dev.ptr(out), dev.ptr(qd), dev.ptr(kd), dev.ptr(vd), b, t, s,
                  h, hkv, d, scale, int(causal), soft_cap, window)
    else:
        rocm.call("aljabr_rocm_fa4_attention", dev.ptr(out), dev.ptr(qd), dev.ptr(kd), dev.ptr(vd), b, t, s, h, hkv,
                  d, scale, int(causal), 0, soft_cap)
    return dev.get(out).reshape(q.shape)


CASES = [
    # b, t, s, h, hkv, d, causal
    (1, 128, 128, 8, 2, 128, True),     # one query block, four full tiles
    (1, 300, 300, 4, 1, 128, True),     # partial block and tile
    (2, 96, 96, 8, 8, 64, True),        # MHA, D = 64, two batches
    (1, 64, 500, 8, 1, 128, True),      # chunked prefill: S > T, bottom-right limit
    (1, 200, 70, 4, 2, 128, True),      # T > S
    (1, 130, 257, 16, 2, 64, False),    # non-causal, G = 8
    (1, 1, 333, 8, 2, 128, True),       # one query row
    (3, 33, 40, 2, 2, 64, True),
    # grids of at least four workgroups per CU take two 32-row tiles per wave
    (8, 300, 300, 64, 8, 128, True),
    (8, 260, 400, 64, 16, 64, True),
]


@pytest.mark.parametrize("b,t,s,h,hkv,d,causal", CASES)
def test_fa4_matches_oracle(rocm, dev, oracle, b, t, s, h, hkv, d, causal):
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=7 + t + s + d)
    scale = 1.0 / np.sqrt(d)
    got = _run(rocm, dev, q, k, v, scale, causal)
    ref = oracle.fa4_attention(q, k, v, scale=scale, causal=causal)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= TOL
    # every (row, head) on its own
    err = np.linalg.norm((got - ref).reshape(-1, d), axis=1) / np.maximum(np.linalg.norm(ref.reshape(-1, d), axis=1),
                                                                          1e-30)
    assert err.max() <= 5 * TOL


@pytest.mark.parametrize("cap", [1.0, 30.0])
def test_fa4_soft_cap(rocm, dev, oracle, cap):
    q, k, v = _qkv(oracle, 1, 150, 150, 4, 2, 128, seed=91)
    q *= 3.0                                    # scores well into the cap
    got = _run(rocm, dev, q, k, v, 0.2, True, soft_cap=cap)
    ref = oracle.fa4_attention(q, k, v, scale=0.2, causal=True, soft_cap=cap)
    assert rel_l2(got, ref) <= TOL


# window 20: the second query block's keys start in tile 3 (an odd first tile).
@pytest.mark.parametrize("window", [1, 17, 20, 64, 1000])
def test_fa4_window(rocm, dev, oracle, window):
    q, k, v = _qkv(oracle, 1, 200, 230, 4, 2, 128, seed=101)
    got = _run(rocm, dev, q, k, v, 0.09, True, window=window)
    ref = oracle.fa4_attention(q, k, v, scale=0.09, causal=True, window=window)
    assert rel_l2(got, ref) <= TOL
    # T = S: row t sees keys max(t + 1 - window, 0) .. t
    q2, k2, v2 = _qkv(oracle, 2, 200, 200, 8, 2, 64, seed=103)
    got = _run(rocm, dev, q2, k2, v2, 0.125, True, window=window)
    assert rel_l2(got, oracle.fa4_attention(q2, k2, v2, scale=0.125, causal=True, window=window)) <= TOL


@pytest.mark.parametrize("d", [2, 48, 80, 256])
def test_fa4_generic_head_sizes(rocm, dev, oracle, d):
    q, k, v = _qkv(oracle, 1, 40, 1500, 4, 2, d, seed=3 + d)   # S > one LDS chunk of keys
    got = _run(rocm, dev, q, k, v, 1.0 / np.sqrt(d), True)
    ref = oracle.fa4_attention(q, k, v, scale=1.0 / np.sqrt(d), causal=True)
    assert rel_l2(got, ref) <= TOL


def test_fa4_unaligned_pointers_take_the_generic_kernel(rocm, dev, oracle):
    import torch
    b, t, s, h, hkv, d = 1, 50, 60, 4, 2, 128
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=55)
    buf = [dev.put(np.concatenate([np.zeros(1, np.float32), a.ravel()])) for a in (q, k, v)]
    out = torch.zeros(q.size + 1, dtype=torch.float32, device="cuda:0")
    ptr = [x.data_ptr() + 4 for x in buf]
    rocm.call("aljabr_rocm_fa4_attention", out.data_ptr() + 4, ptr[0], ptr[1], ptr[2], b, t, s, h, hkv, d,
              0.1, 1, 0, 0.0)
    got = dev.get(out)[1:].reshape(q.shape)
    assert rel_l2(got, oracle.fa4_attention(q, k, v, scale=0.1, causal=True)) <= TOL


def test_fa4_reference_uniform_fixture(rocm, dev, oracle):
    """FlashAttentionCpuTest.java:12-35 (zero Q and K, V[i] = (2i, 2i+1), 65
    keys): every row is the mean of V, on the generic (D = 2) and the
    matrix-core (D = 64, zero-padded) kernels."""
    v2 = np.arange(130, dtype=np.float32).reshape(1, 65, 1, 2)
    mean = v2.reshape(65, 2).astype(np.float64).mean(axis=0)
    z2 = np.zeros_like(v2)
    got = _run(rocm, dev, z2, z2, v2, 1.0 / np.sqrt(2.0), False)
    np.testing.assert_allclose(got.reshape(65, 2), np.broadcast_to(mean, (65, 2)), atol=1e-4)
    v64 = np.zeros((1, 65, 1, 64), np.float32)
    v64[..., :2] = v2
    z64 = np.zeros_like(v64)
    got = _run(rocm, dev, z64, z64, v64, 0.125, False)
    np.testing.assert_allclose(got[0, :, 0, :2], np.broadcast_to(mean, (65, 2)), atol=1e-3)
    assert np.abs(got[..., 2:]).max() == 0.0


def test_fa4_llama3_8b_prefill_rows(rocm, dev, oracle):
    """T = S = 2048, 32 query heads over 8 KV heads, D = 128, causal: sampled
    rows equal one-row oracle problems over their visible keys (row t sees
    keys 0..t)."""
    b, t, s, h, hkv, d = 1, 2048, 2048, 32, 8, 128
    q, k, v = _qkv(oracle, b, t, s, h, hkv, d, seed=2024)
    scale = 1.0 / np.sqrt(d)
    got = _run(rocm, dev, q, k, v, scale, True)
    assert np.isfinite(got).all()
    rng = np.random.default_rng(5)
    rows = sorted(set([0, 1, 31, 32, 127, 128, 1023, 2047] + list(rng.integers(0, t, 8))))
    for row in rows:
        ref = oracle.fa4_attention(q[:, row:row + 1], k[:, :row + 1], v[:, :row + 1], scale=scale, causal=False)
        assert rel_l2(got[:, row], ref[:, 0]) <= TOL, row


def test_fa4_argument_errors(rocm, dev):
    from aljabr_amd import abi
    x = dev.empty(64)
    with pytest.raises(abi.RocmError) as e:
        rocm.call("aljabr_rocm_fa4_attention", dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), 1, 1, 1, 3, 2, 8,
                  1.0, 1, 0, 0.0)
    assert e.value.status == abi.ERR_BAD_ARGUMENT
    with pytest.raises(abi.RocmError) as e:
        rocm.call("aljabr_rocm_fa4_attention", None, dev.ptr(x), dev.ptr(x), dev.ptr(x), 1, 1, 1, 1, 1, 8,
                  1.0, 1, 0, 0.0)
    assert e.value.status == abi.ERR_BAD_ARGUMENT
    with pytest.raises(abi.RocmError) as e:
        rocm.call("aljabr_rocm_fa4_attention", dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), 1, 1, 1, 1, 1, 512,
                  1.0, 1, 0, 0.0)
    assert e.value.status == abi.ERR_UNSUPPORTED
    assert rocm.load().aljabr_rocm_fa4_sdpa_available() == 1
    assert rocm.load().aljabr_rocm_fa4_bf16_available() == 0
