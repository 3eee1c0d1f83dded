"""GPU parity for GQA attention (split-K online softmax) against the oracle's
restatement of CpuBackend.attentionGqa: the reference's known answers, the
BASELINE decode configs (Hq 32 / Hkv 8 / D 128, fp16 K/V), masks, causal
alignment and prefill-shaped queries. Tolerance: relative L2 <= 1e-3."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _f(v):
    return {"-inf": -np.inf, "inf": np.inf, "nan": np.nan}.get(v, v) if isinstance(v, str) else v


def _arr(xs):
    return np.array([_f(v) for v in xs], dtype=np.float32)


def run(rocm, dev, q, k, v, mask=None, causal=False, kv_f16=False):
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    qd = dev.put(q.astype(np.float32))
    if kv_f16:
        kd, vd = dev.put(k.astype(np.float16).view(np.uint16)), dev.put(v.astype(np.float16).view(np.uint16))
    else:
        kd, vd = dev.put(k.astype(np.float32)), dev.put(v.astype(np.float32))
    md = dev.put(mask.astype(np.float32)) if mask is not None else None
    out = dev.empty(q.size)
    rocm.call("aljabr_rocm_attention_gqa", dev.ptr(out), dev.ptr(qd), dev.ptr(kd), dev.ptr(vd),
              dev.ptr(md) if md is not None else None, b, hq, hkv, sq, sk, d,
              rocm.TYPE_F16 if kv_f16 else rocm.TYPE_F32, 0.0, int(causal))
    return dev.get(out).reshape(q.shape)


@pytest.mark.parametrize("case", KATS["attention"], ids=lambda c: c["source"])
def test_reference_known_answers(rocm, dev, case):
    q = _arr(case["q"]).reshape(case["q_shape"])
    k = _arr(case["k"]).reshape(case["k_shape"])
    v = _arr(case["v"]).reshape(case["k_shape"])
    mask = None if case["mask"] is None else _arr(case["mask"]).reshape(case["q_shape"][2], case["k_shape"][2])
    out = run(rocm, dev, q, k, v, mask, case["causal"])
    assert np.allclose(out.ravel(), np.array(case["expected"]), atol=case["tolerance"], rtol=0)


@pytest.mark.parametrize("case", KATS["attention_rejects"], ids=lambda c: c["source"])
def test_rejects_bad_masks(rocm, dev, case):
    q = np.zeros((1, 1, 2, 1), np.float32)
    kv = np.array([2.0, 8.0], np.float32).reshape(1, 1, 2, 1)
    with pytest.raises(rocm.RocmError) as e:
        run(rocm, dev, q, np.zeros_like(kv), kv, _arr(case["mask"]).reshape(2, 2), case["causal"])
    assert e.value.status == rocm.ERR_BAD_ARGUMENT


def _inputs(oracle, b, hq, hkv, sq, sk, d, seed):
    q = oracle.normal(seed, b * hq * sq * d).reshape(b, hq, sq, d)
    k = oracle.normal(seed + 1, b * hkv * sk * d).reshape(b, hkv, sk, d)
    v = oracle.normal(seed + 2, b * hkv * sk * d).reshape(b, hkv, sk, d)
    # K/V are fp16 in the configs: round them once so both sides see the same values.
    return q, k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("b,s", [(1, 512), (1, 4096), (1, 32768), (16, 512), (16, 4096), (64, 512)])
def test_decode_configs_fp16_kv(rocm, dev, oracle, b, s):
    q, k, v = _inputs(oracle, b, 32, 8, 1, s, 128, seed=b * 100003 + s)
    ref = oracle.attention_gqa(q, k, v, None, True)
    out = run(rocm, dev, q, k, v, None, True, kv_f16=True)
    assert rel_l2(out, ref) <= TOL


@pytest.mark.parametrize("g", [1, 2, 4, 8])
@pytest.mark.parametrize("d", [64, 128])
def test_head_groupings_fp32_kv(rocm, dev, oracle, g, d):
    hkv = 4
    q, k, v = _inputs(oracle, 2, hkv * g, hkv, 1, 700, d, seed=g * 10 + d)
    ref = oracle.attention_gqa(q, k, v, None, False)
    out = run(rocm, dev, q, k, v)
    assert rel_l2(out, ref) <= TOL


def test_prefill_shaped_query_with_mask_and_causal(rocm, dev, oracle):
    q, k, v = _inputs(oracle, 2, 8, 2, 5, 300, 128, seed=77)
    rng = np.random.default_rng(1)
    mask = rng.normal(0, 1, (5, 300)).astype(np.float32)
    mask[rng.random((5, 300)) < 0.2] = -np.inf
    mask[4, :] = -np.inf                                      # a fully masked row -> zeros
    ref = oracle.attention_gqa(q, k, v, mask, True)
    out = run(rocm, dev, q, k, v, mask, True)
    assert rel_l2(out, ref) <= TOL
    assert np.all(out[:, :, 4] == 0)


def test_more_queries_than_keys_gives_zero_rows(rocm, dev, oracle):
    q, k, v = _inputs(oracle, 1, 4, 4, 6, 3, 128, seed=5)
    ref = oracle.attention_gqa(q, k, v, None, True)
    out = run(rocm, dev, q, k, v, None, True)
    assert np.all(out[:, :, :3] == 0) and rel_l2(out, ref) <= TOL


# BASELINE configs[3] points too large for the oracle over every head: fp16
# K/V generated on the device (8 GiB at B=64, S=32768), three (batch,
# kv-head) groups checked against the oracle on their slices, and every
# output row a convex combination of V (finite, bounded).
@pytest.mark.parametrize("b,s", [(64, 32768), (16, 32768), (64, 4096)], ids=["b64-s32768", "b16-s32768",
                                                                          "b64-s4096"])
def test_full_size_spot_rows(rocm, dev, oracle, b, s):
    import torch
    hq, hkv, d = 32, 8, 128
    print(f"\n[attention full size] B={b} S={s}", flush=True)
    gen = torch.Generator(device="cuda:0").manual_seed(1234 + b + s)
    k = torch.randn((b, hkv, s, d), generator=gen, device="cuda:0", dtype=torch.float16)
    v = torch.randn((b, hkv, s, d), generator=gen, device="cuda:0", dtype=torch.float16)
    q = torch.randn((b, hq, 1, d), generator=gen, device="cuda:0", dtype=torch.float32)
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    rocm.call("aljabr_rocm_attention_gqa", out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), None,
              b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o))
    vmax = float(v.abs().max().item())
    assert np.abs(o).max() <= vmax + 1e-3
    for bi, kvh in [(0, 0), (b // 2 - 1, 5), (b - 1, 7)]:
        ks = k[bi:bi + 1, kvh:kvh + 1].float().cpu().numpy()
        vs = v[bi:bi + 1, kvh:kvh + 1].float().cpu().numpy()
        qs = q[bi:bi + 1, kvh * 4:(kvh + 1) * 4].cpu().numpy()
        ref = oracle.attention_gqa(qs, np.ascontiguousarray(ks), np.ascontiguousarray(vs), None, True)
        assert rel_l2(o[bi:bi + 1, kvh * 4:(kvh + 1) * 4], ref) <= TOL
    del k, v
    torch.cuda.empty_cache()


# ---- paged KV (the Metal bridge's ABI) -------------------------------------

def _paged_inputs(oracle, b, t, h, hkv, d, bs, mb, ctx, seed):
    q = oracle.normal(seed, b * t * h * d).reshape(b, t, h, d)
    kc = oracle.normal(seed + 1, b * mb * hkv * bs * d).reshape(b * mb, hkv, bs, d)
    vc = oracle.normal(seed + 2, b * mb * hkv * bs * d).reshape(b * mb, hkv, bs, d)
    table = np.random.default_rng(seed).permutation(b * mb).astype(np.int32).reshape(b, mb)
    return q, kc, vc, table, np.array(ctx, np.int32)


def run_paged(rocm, dev, q, kc, vc, table, cl, scale, causal=1, qsp=0, window=0, cap=0.0, fill=np.nan):
    b, t, h, d = q.shape
    hkv, bs = kc.shape[1], kc.shape[2]
    out = dev.put(np.full(q.size, fill, np.float32))
    # Keep every device buffer referenced until the call returns: a freed
    # temporary's memory is handed to the next upload.
    bufs = [dev.put(a) for a in (q, kc, vc, table, cl)]
    args = [dev.ptr(out)] + [dev.ptr(t_) for t_ in bufs] + [b, t, h, hkv, d, bs, table.shape[1], scale, causal]
    if qsp or window:
        rocm.call("aljabr_rocm_paged_attention_gqa_windowed", *args, qsp, window, cap)
    else:
        rocm.call("aljabr_rocm_paged_attention_gqa", *args, cap)
    return dev.get(out).reshape(q.shape)


# (B, T, H, Hkv, D, block size, max blocks, context lengths, causal, query start, window, soft cap):
# decode and short prefill rows, every split-kernel grouping and the generic
# kernel (D = 80), ragged and empty contexts, windows and soft caps.
PAGED = [
    (1, 1, 32, 8, 128, 16, 130, [2049], 1, 0, 0, 0.0),
    (3, 1, 32, 8, 128, 32, 20, [600, 0, 17], 1, 0, 0, 0.0),
    (2, 4, 8, 8, 64, 16, 12, [150, 5], 1, 0, 0, 30.0),
    (2, 1, 16, 2, 128, 16, 40, [613, 301], 1, 612, 64, 0.0),
    (1, 3, 8, 1, 64, 8, 16, [100], 0, 0, 0, 0.0),
    (2, 2, 12, 4, 80, 16, 8, [100, 33], 1, 0, 0, 5.0),
]


@pytest.mark.parametrize("case", PAGED, ids=[f"paged{i}" for i in range(len(PAGED))])
def test_paged_attention_matches_oracle(rocm, dev, oracle, case):
    b, t, h, hkv, d, bs, mb, ctx, causal, qsp, window, cap = case
    q, kc, vc, table, cl = _paged_inputs(oracle, b, t, h, hkv, d, bs, mb, ctx, seed=sum(ctx) + d)
    scale = 1.0 / np.sqrt(d)
    rc, ref = oracle.paged_attention(q, kc, vc, table, cl, scale, causal, qsp, window, cap)
    assert rc == 0
    out = run_paged(rocm, dev, q, kc, vc, table, cl, scale, causal, qsp, window, cap)
    assert rel_l2(out, ref) <= TOL
    for bi, c in enumerate(ctx):
        if c <= 0:
            assert np.all(out[bi] == 0)


def test_paged_attention_zero_length_context_zero_fills(rocm, dev, oracle):
    """MetalBindingNativeFallbackTest.nativeAttentionZeroLengthContextZeroFillsOutput
    (backend/metal/.../MetalBindingNativeFallbackTest.java:109-150): out starts at 42."""
    q = np.ones((1, 2, 1, 64), np.float32)
    kc = np.zeros((1, 1, 4, 64), np.float32)
    out = run_paged(rocm, dev, q, kc, kc, np.zeros((1, 1), np.int32), np.zeros(1, np.int32), 1.0, fill=42.0)
    assert np.array_equal(out, np.zeros_like(out))


def test_paged_attention_statuses(rocm, dev, oracle):
    q, kc, vc, table, cl = _paged_inputs(oracle, 1, 1, 8, 2, 64, 16, 4, [40], seed=3)
    bufs = [dev.put(a) for a in (q, q, kc, vc, table, cl)]
    with pytest.raises(rocm.RocmError) as e:           # H not a multiple of H_kv: -1, as the Metal bridge
        rocm.call("aljabr_rocm_paged_attention_gqa", *[dev.ptr(t_) for t_ in bufs], 1, 1, 8, 3, 64, 16, 4,
                  0.125, 1, 0.0)
    assert e.value.status == -1
    bad = table.copy()
    bad[0, 1] = -4                                     # a block the context uses
    with pytest.raises(rocm.RocmError) as e:
        run_paged(rocm, dev, q, kc, vc, bad, cl, 0.125)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:           # 65 keys need 5 blocks of 16, the table has 4
        run_paged(rocm, dev, q, kc, vc, table, np.array([65], np.int32), 0.125)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    bad[0, 3] = -1                                     # unused entries are not checked
    bad[0, 1] = table[0, 1]
    out = run_paged(rocm, dev, q, kc, vc, bad, np.array([40], np.int32), 0.125)
    rc, ref = oracle.paged_attention(q, kc, vc, bad, np.array([40], np.int32), 0.125)
    assert rc == 0 and rel_l2(out, ref) <= TOL
