"""Pins the CPU oracle (CPU only, no GPU calls).

Each oracle function is checked against the reference's own known answers
(tests/golden/reference_kats.json, transcribed from its JUnit tests) and, where
those leave gaps, against what the mathematics fixes: exhaustive comparison
with IEEE binary16, closed forms, invariants and float64 brute force. The
checks are chosen so that a plausible mistake (swapped nibbles, a dropped
+0.0f, ties rounded the wrong way, a transposed operand) fails one of them.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

from conftest import rel_l2

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def _f(v):
    return {"-inf": -np.inf, "inf": np.inf, "nan": np.nan}.get(v, v) if isinstance(v, str) else v


def _arr(xs):
    return np.array([_f(v) for v in xs], dtype=np.float32)


# ---------------------------------------------------------------- conversions

def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    expected = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(expected)
    # Every NaN decodes to the canonical quiet NaN (GgufQuantTables.java:160).
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


def test_writer_half_rounding(oracle):
    rng = np.random.default_rng(7)
    vals = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 1e-3, 2000), rng.normal(0, 1e-6, 500)]).astype(np.float32)
    for v in vals:
        bits = int(np.float32(v).view(np.uint32))
        got = oracle.f32_to_f16_writer(float(v))
        rne = int(np.float16(v).view(np.uint16))
        # Mantissa remainder exactly half way -> writer rounds up in magnitude.
        exp = ((bits >> 23) & 0xFF) - 127 + 15
        if exp > 0:
            tie = (bits & 0x1FFF) == 0x1000
        else:
            shift = 14 - exp
            full = (bits & 0x7FFFFF) | 0x800000
            tie = exp >= -10 and (full & ((1 << shift) - 1)) == (1 << (shift - 1))
        if not tie:
            assert got == rne, (v, hex(got), hex(rne))
    # Closed-form cases.
    assert oracle.f32_to_f16_writer(1.0) == 0x3C00
    assert oracle.f32_to_f16_writer(-2.0) == 0xC000
    assert oracle.f32_to_f16_writer(1.0 + 2.0 ** -11) == 0x3C01      # tie -> up (RNE would give 0x3C00)
    assert oracle.f32_to_f16_writer(1.0 + 3 * 2.0 ** -11) == 0x3C02  # tie -> up (RNE agrees)
    assert oracle.f32_to_f16_writer(2.0 ** -24) == 0x0001              # smallest subnormal
    assert oracle.f32_to_f16_writer(2.0 ** -26) == 0x0000              # below the subnormal range
    assert oracle.f32_to_f16_writer(70000.0) == 0x7C01                 # overflow with mantissa bits set
    assert oracle.f32_to_f16_writer(65536.0) == 0x7C00                 # overflow, zero mantissa -> inf


def test_java_round(oracle):
    cases = {0.5: 1, -0.5: 0, 1.5: 2, -1.5: -1, 2.5: 3, -2.5: -2, 0.49999997: 0, -0.49999997: 0,
             7.4999995: 7, 1e10: 2147483647, -1e10: -2147483648, float("nan"): 0}
    for v, r in cases.items():
        assert oracle.java_round(v) == r, v


# ---------------------------------------------------------------------- Q4_0

def test_q4_0_known_rows(oracle):
    k = KATS["q4_0_rows"]
    blocks = np.array(k["blocks"], dtype=np.uint8)
    w = oracle.dequant(oracle.QTYPE_Q4_0, blocks, 64).reshape(2, 32)
    assert np.array_equal(w[0], np.array(k["row0"], dtype=np.float32))
    ones = np.ones(32, dtype=np.float32)
    for r in range(2):
        assert oracle.dot_row(oracle.QTYPE_Q4_0, blocks[r * 18:(r + 1) * 18], ones) == k["dot_ones"][r]
    y = oracle.q_matvec(oracle.QTYPE_Q4_0, blocks, ones, 2, 32, nthreads=1)
    assert list(y) == k["dot_ones"]


def test_q4_0_lane_order(oracle):
    k = KATS["q4_0_lane_order"]
    blk = np.array([k["scale_bits"] & 0xFF, k["scale_bits"] >> 8] + k["codes"], dtype=np.uint8)
    w = oracle.dequant(oracle.QTYPE_Q4_0, blk, 32)
    assert np.array_equal(w, np.array(k["expected_row"], dtype=np.float32))


def test_q4_0_zero_code_negative_scale_is_positive_zero(oracle):
    # (q-8)*d + 0.0f with q=8 and d<0 is +0.0 (GgufBlockDequantizer.java:414-415).
    blk = np.array([0x00, 0xBC] + [0x88] * 16, dtype=np.uint8)   # d = -1.0, every code 8
    w = oracle.dequant(oracle.QTYPE_Q4_0, blk, 32)
    assert np.all(w.view(np.uint32) == 0)


def test_q4_0_raw_pattern(oracle):
    k = KATS["q4_0_raw_pattern"]
    blocks = []
    for h, p in zip(k["half_scales"], k["packed"]):
        blocks += [h & 0xFF, h >> 8] + [p] * 16
    blocks = np.array(blocks, dtype=np.uint8)
    vec = np.array(k["vector"], dtype=np.float32)
    # The test's scalar reference (GgufQ32RawTest.java:221-235).
    ref = np.float32(0)
    for b, (s, p) in enumerate(zip(k["scales"], k["packed"])):
        lo, hi = p & 15, p >> 4
        for i in range(16):
            ref = np.float32(ref + np.float32(s) * np.float32(lo - 8) * vec[32 * b + i])
            ref = np.float32(ref + np.float32(s) * np.float32(hi - 8) * vec[32 * b + 16 + i])
    got = oracle.dot_row(oracle.QTYPE_Q4_0, blocks, vec)
    assert abs(got - float(ref)) <= k["tolerance"]


def test_q4_0_encoder_known_block(oracle):
    # Hand-worked GGUFWriter.encodeQ4_0 block: maxAbs 7 -> scale 1.0 exactly.
    w = np.zeros(32, dtype=np.float32)
    w[0], w[16], w[1], w[17], w[2] = 7.0, -7.0, 2.5, -2.5, 0.49
    enc = oracle.quantize(oracle.QTYPE_Q4_0, w)
    assert enc[0] == 0x00 and enc[1] == 0x3C
    # byte i = (round(w[16+i])+8) << 4 | (round(w[i])+8); Math.round(2.5)=3, round(-2.5)=-2.
    assert enc[2] == ((-7 + 8) << 4 | (7 + 8))
    assert enc[3] == ((-2 + 8) << 4 | (3 + 8))
    assert enc[4] == ((0 + 8) << 4 | (0 + 8))
    # -8 is reachable only by clamping: -8.0 would need scale 8/8.
    w2 = np.zeros(32, dtype=np.float32); w2[0] = -7.0; w2[1] = 7.0
    enc2 = oracle.quantize(oracle.QTYPE_Q4_0, w2)
    assert enc2[2] & 15 == 1 and enc2[3] & 15 == 15


def test_q4_0_round_trip_error_bound(oracle):
    w = oracle.normal(101, 32 * 512, 0.0, 0.02)
    enc = oracle.quantize(oracle.QTYPE_Q4_0, w)
    dec = oracle.dequant(oracle.QTYPE_Q4_0, enc, w.size)
    blocks = w.reshape(-1, 32)
    scale = np.abs(blocks).max(axis=1) / 7.0
    err = np.abs(dec.reshape(-1, 32) - blocks)
    # half a quantization step plus the fp16 rounding of the stored scale.
    assert np.all(err <= (0.5 * scale + 8 * scale * 2.0 ** -10)[:, None] + 1e-12)


def test_q4_0_matvec_vs_float64(oracle):
    n, k = 64, 256
    w = oracle.normal(5, n * k, 0.0, 0.02)
    x = oracle.normal(6, k)
    enc = oracle.quantize(oracle.QTYPE_Q4_0, w)
    dense = oracle.dequant(oracle.QTYPE_Q4_0, enc, n * k).reshape(n, k).astype(np.float64)
    y = oracle.q_matvec(oracle.QTYPE_Q4_0, enc, x, n, k)
    assert rel_l2(y, dense @ x.astype(np.float64)) < 1e-6
    # Catches a transposed operand: x against columns would not match.
    assert rel_l2(y, dense[:, :n].T @ x[:n].astype(np.float64)) > 0.1


# ---------------------------------------------------------------------- Q8_0

def test_q8_0_known_rows(oracle):
    k = KATS["q8_0_rows"]
    blocks = np.array(k["blocks"], dtype=np.uint8)
    ones = np.ones(32, dtype=np.float32)
    y = oracle.q_matvec(oracle.QTYPE_Q8_0, blocks, ones, 2, 32, nthreads=1)
    assert list(y) == k["dot_ones"]


def test_q8_0_raw_pattern(oracle):
    k = KATS["q8_0_raw_pattern"]
    blocks = np.array(k["blocks"], dtype=np.uint8)
    vec = np.array(k["vector"], dtype=np.float32)
    off = k["vector_offset"]
    ref = np.float32(0)
    for b, (s, seed) in enumerate(zip(k["scales"], k["seeds"])):
        for i in range(32):
            q = np.int8(np.uint8((seed + 41 * i) & 0xFF).view(np.int8))
            ref = np.float32(ref + np.float32(s) * np.float32(q) * vec[off + 32 * b + i])
    got = oracle.dot_row(oracle.QTYPE_Q8_0, blocks, np.ascontiguousarray(vec[off:]))
    assert abs(got - float(ref)) <= k["tolerance"]
    # The decoder agrees: sum of decoded weights times x.
    dec = oracle.dequant(oracle.QTYPE_Q8_0, blocks, 160)
    assert abs(float(np.dot(dec.astype(np.float64), vec[off:].astype(np.float64))) - float(ref)) <= k["tolerance"]


def test_q8_0_encoder(oracle):
    w = np.zeros(32, dtype=np.float32)
    w[0], w[1], w[2] = 127.0, -63.5, 0.5
    enc = oracle.quantize(oracle.QTYPE_Q8_0, w)
    assert enc[0] == 0x00 and enc[1] == 0x3C          # scale 1.0
    assert enc[2] == 127 and enc[3] == np.uint8(-63 & 0xFF) and enc[4] == 1   # round(-63.5) = -63
    w2 = oracle.normal(9, 32 * 256, 0.0, 0.02)
    dec = oracle.dequant(oracle.QTYPE_Q8_0, oracle.quantize(oracle.QTYPE_Q8_0, w2), w2.size)
    scale = np.abs(w2.reshape(-1, 32)).max(axis=1) / 127.0
    err = np.abs(dec - w2).reshape(-1, 32)
    assert np.all(err <= (0.5 * scale + 127 * scale * 2.0 ** -10)[:, None] + 1e-12)


# ----------------------------------------------------------------------- NF4

def test_nf4_table_is_the_reference_codebook(oracle):
    assert oracle.NF4_TABLE[7] == 0.0 and oracle.NF4_TABLE[0] == -1.0 and oracle.NF4_TABLE[15] == 1.0
    assert np.all(np.diff(oracle.NF4_TABLE) > 0)


def test_nf4_dequant_closed_form(oracle):
    rng = np.random.default_rng(3)
    numel, group = 1024, 64
    codes = rng.integers(0, 256, numel // 2, dtype=np.uint8)
    absmax = rng.uniform(0.001, 0.1, numel // group).astype(np.float32)
    absmax[0] = 0.0
    got = oracle.nf4_dequant(codes, absmax, numel, group)
    hi, lo = codes >> 4, codes & 15
    nib = np.stack([hi, lo], axis=1).ravel()           # even element = high nibble
    exp = (oracle.NF4_TABLE[nib] * np.repeat(absmax, group)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    # Swapped nibble order would differ.
    swapped = (oracle.NF4_TABLE[np.stack([lo, hi], axis=1).ravel()] * np.repeat(absmax, group)).astype(np.float32)
    assert not np.array_equal(got, swapped)
    # Special cases.
    assert np.all(got[:group] == 0)
    # code 0 -> -absmax, code 7 -> 0, code 15 -> +absmax
    one = oracle.nf4_dequant(np.array([0x07, 0xF0], dtype=np.uint8), np.array([0.5], dtype=np.float32), 4, 64)
    assert list(one) == [-0.5, 0.0, 0.5, -0.5]


def test_nf4_odd_numel_ignores_last_low_nibble(oracle):
    got = oracle.nf4_dequant(np.array([0xF0, 0xFF], dtype=np.uint8), np.array([2.0], dtype=np.float32), 3, 64)
    assert list(got) == [2.0, -2.0, 2.0]


def test_nf4_quantize_picks_nearest_level(oracle):
    w = oracle.normal(11, 64 * 300, 0.0, 0.02)
    codes, absmax = oracle.nf4_quantize(w, 64)
    assert np.array_equal(absmax, np.abs(w.reshape(-1, 64)).max(axis=1))
    dec = oracle.nf4_dequant(codes, absmax, w.size, 64)
    norm = (w.reshape(-1, 64) / absmax[:, None]).ravel().astype(np.float32)
    dist = np.abs(norm[:, None].astype(np.float64) - oracle.NF4_TABLE[None, :].astype(np.float64))
    best = dist.min(axis=1)
    hi, lo = codes >> 4, codes & 15
    chosen = np.stack([hi, lo], axis=1).ravel()
    assert np.allclose(dist[np.arange(w.size), chosen], best, atol=1e-7)
    assert np.allclose(dec, oracle.NF4_TABLE[chosen] * np.repeat(absmax, 64), atol=0)


def test_nf4_matvec_vs_float64(oracle):
    n, k, g = 96, 512, 64
    w = oracle.normal(21, n * k, 0.0, 0.02)
    codes, absmax = oracle.nf4_quantize(w, g)
    dense = oracle.nf4_dequant(codes, absmax, n * k, g).reshape(n, k).astype(np.float64)
    for m in (1, 3):
        x = oracle.normal(22 + m, m * k)
        y = oracle.nf4_matvec(codes, absmax, x, n, k, g)
        assert rel_l2(y, (x.reshape(m, k).astype(np.float64) @ dense.T).reshape(y.shape)) < 1e-6


def test_f16_matvec_vs_float64(oracle):
    n, k = 40, 96
    w = oracle.normal(31, n * k).astype(np.float16)
    x = oracle.normal(32, k)
    y = oracle.f16_matvec(w.view(np.uint16), x, n, k)
    assert rel_l2(y, w.astype(np.float64).reshape(n, k) @ x.astype(np.float64)) < 1e-6


# ----------------------------------------------------------------- attention

@pytest.mark.parametrize("case", KATS["attention"], ids=lambda c: c["source"])
def test_attention_known_answers(oracle, case):
    q = _arr(case["q"]).reshape(case["q_shape"])
    k = _arr(case["k"]).reshape(case["k_shape"])
    v = _arr(case["v"]).reshape(case["k_shape"])
    mask = None if case["mask"] is None else _arr(case["mask"]).reshape(case["q_shape"][2], case["k_shape"][2])
    out = oracle.attention_gqa(q, k, v, mask, case["causal"], nthreads=1)
    assert np.allclose(out.ravel(), np.array(case["expected"], dtype=np.float64), atol=case["tolerance"], rtol=0)


@pytest.mark.parametrize("case", KATS["attention_rejects"], ids=lambda c: c["source"])
def test_attention_rejects_bad_masks(oracle, case):
    q = np.zeros((1, 1, 2, 1), np.float32)
    kv = np.array([2.0, 8.0], np.float32).reshape(1, 1, 2, 1)
    with pytest.raises(ValueError):
        oracle.attention_gqa(q, np.zeros_like(kv), kv, _arr(case["mask"]).reshape(2, 2), case["causal"])


def test_attention_vs_float64_softmax(oracle):
    b, hq, hkv, sq, sk, d = 2, 8, 2, 3, 37, 16
    q = oracle.normal(41, b * hq * sq * d).reshape(b, hq, sq, d)
    k = oracle.normal(42, b * hkv * sk * d).reshape(b, hkv, sk, d)
    v = oracle.normal(43, b * hkv * sk * d).reshape(b, hkv, sk, d)
    out = oracle.attention_gqa(q, k, v, None, True)
    ref = np.zeros_like(out, dtype=np.float64)
    for bi in range(b):
        for h in range(hq):
            kv = h // (hq // hkv)
            for qi in range(sq):
                lim = min(sk, sk - sq + qi + 1)
                s = (k[bi, kv, :lim].astype(np.float64) @ q[bi, h, qi].astype(np.float64)) / math.sqrt(d)
                p = np.exp(s - s.max())
                ref[bi, h, qi] = (p / p.sum()) @ v[bi, kv, :lim].astype(np.float64)
    assert rel_l2(out, ref) < 1e-5
    # identical keys -> mean of the visible values (closed form)
    kk = np.repeat(k[:, :, :1], sk, axis=2)
    out2 = oracle.attention_gqa(q, kk, v, None, False)
    assert np.allclose(out2[0, 0, 0], v[0, 0].mean(axis=0), atol=1e-5)


def _paged_case(oracle, b, t, h, hkv, d, bs, max_blocks, ctx, seed):
    """Random q and a contiguous K/V per sequence, scattered into physical
    blocks through a random permutation."""
    q = oracle.normal(seed, b * t * h * d).reshape(b, t, h, d)
    kv_len = max_blocks * bs
    k = oracle.normal(seed + 1, b * hkv * kv_len * d).reshape(b, hkv, kv_len, d)
    v = oracle.normal(seed + 2, b * hkv * kv_len * d).reshape(b, hkv, kv_len, d)
    perm = np.random.default_rng(seed).permutation(b * max_blocks).astype(np.int32)
    table = perm.reshape(b, max_blocks)
    kc = np.zeros((b * max_blocks, hkv, bs, d), np.float32)
    vc = np.zeros_like(kc)
    for bi in range(b):
        for blk in range(max_blocks):
            kc[table[bi, blk]] = k[bi, :, blk * bs:(blk + 1) * bs]
            vc[table[bi, blk]] = v[bi, :, blk * bs:(blk + 1) * bs]
    return q, k, v, kc, vc, table, np.array(ctx, np.int32)


def test_paged_attention_zero_length_context_zero_fills(oracle):
    """MetalBindingNativeFallbackTest.nativeAttentionZeroLengthContextZeroFillsOutput
    (backend/metal/.../MetalBindingNativeFallbackTest.java:109-150)."""
    q = np.ones((1, 2, 1, 2), np.float32)
    kc = np.zeros((1, 1, 4, 2), np.float32)
    rc, out = oracle.paged_attention(q, kc, kc, np.zeros((1, 1), np.int32), np.zeros(1, np.int32), 1.0, True)
    assert rc == 0 and np.array_equal(out, np.zeros_like(out))


def test_paged_attention_matches_dense_oracle(oracle):
    """Through any block permutation, causal paged attention without window or
    cap is the dense attention of the (pinned) CpuBackend restatement on the
    first context_len keys, bottom-right aligned."""
    b, t, h, hkv, d, bs, mb = 2, 3, 8, 2, 16, 8, 5
    ctx = [37, 9]
    q, k, v, kc, vc, table, cl = _paged_case(oracle, b, t, h, hkv, d, bs, mb, ctx, 61)
    rc, out = oracle.paged_attention(q, kc, vc, table, cl, 1.0 / math.sqrt(d), True)
    assert rc == 0
    for bi in range(b):
        dense = oracle.attention_gqa(q[bi:bi + 1].transpose(0, 2, 1, 3), k[bi:bi + 1, :, :ctx[bi]],
                                     v[bi:bi + 1, :, :ctx[bi]], None, True)
        assert rel_l2(out[bi], dense[0].transpose(1, 0, 2)) < 1e-5
    # moving the blocks to other physical slots (and the table with them)
    # gives the same bits
    perm = np.random.default_rng(5).permutation(b * mb).astype(np.int32)
    kc3 = np.empty_like(kc)
    vc3 = np.empty_like(vc)
    kc3[perm] = kc
    vc3[perm] = vc
    rc3, out3 = oracle.paged_attention(q, kc3, vc3, perm[table], cl, 1.0 / math.sqrt(d), True)
    assert rc3 == 0 and np.array_equal(out3, out)


def test_paged_attention_window_cap_and_errors(oracle):
    b, t, h, hkv, d, bs, mb = 1, 1, 4, 4, 8, 4, 4
    q, k, v, kc, vc, table, cl = _paged_case(oracle, b, t, h, hkv, d, bs, mb, [13], 71)
    sc = 1.0 / math.sqrt(d)
    # sliding window W at query position 12 (a window disables the bottom-right
    # default, so the position is passed): the last W keys only
    rc, out = oracle.paged_attention(q, kc, vc, table, cl, sc, True, 12, 5)
    dense = oracle.attention_gqa(q.transpose(0, 2, 1, 3), k[:, :, 8:13], v[:, :, 8:13], None, False)
    assert rc == 0 and rel_l2(out, dense.transpose(0, 2, 1, 3)) < 1e-5
    # window 1: exactly the value row of the query position
    rc, out = oracle.paged_attention(q, kc, vc, table, cl, sc, True, 12, 1)
    assert rc == 0 and np.allclose(out[0, 0], v[0, :, 12], atol=1e-6)
    # a cap far above every score changes nothing; identical keys give the mean of V for any cap
    _, base = oracle.paged_attention(q, kc, vc, table, cl, sc, True)
    _, capped = oracle.paged_attention(q, kc, vc, table, cl, sc, True, 0, 0, 1e6)
    assert rel_l2(capped, base) < 1e-6
    kc_same = np.repeat(kc[:, :, :1], bs, axis=2)
    kc_same[:] = kc_same[table[0, 0]]
    _, flat = oracle.paged_attention(q, kc_same, vc, table, cl, sc, True, 0, 0, 0.5)
    assert np.allclose(flat[0, 0], v[0, :, :13].mean(axis=1), atol=1e-5)
    # explicit query position without causal bottom-right alignment
    rc, early = oracle.paged_attention(q, kc, vc, table, cl, sc, True, 3, 0)
    dense = oracle.attention_gqa(q.transpose(0, 2, 1, 3), k[:, :, :4], v[:, :, :4], None, False)
    assert rc == 0 and rel_l2(early, dense.transpose(0, 2, 1, 3)) < 1e-5
    # statuses of aljabr_metal_attention_impl
    assert oracle.paged_attention(q.reshape(1, 1, 4, 8)[:, :, :3], kc, vc, table, cl, sc)[0] == -1
    bad = table.copy()
    bad[0, 2] = -1
    assert oracle.paged_attention(q, kc, vc, bad, cl, sc)[0] == -2
    assert oracle.paged_attention(q, kc, vc, table, np.array([17], np.int32), sc)[0] == -2


# ---------------------------------------------------------- decode-step ops

def test_vector_ops_known_answers(oracle):
    k = KATS["vector_ops"]
    d = k["delta"]
    for c in k["rmsnorm"]:
        out = oracle.rmsnorm(np.array(c["x"], np.float32), np.array(c["w"], np.float32), c["eps"])
        assert np.allclose(out, c["expected"], atol=d, rtol=0)
    assert np.allclose(oracle.softmax(np.array(k["softmax"]["x"], np.float32)), k["softmax"]["expected"], atol=d)
    assert np.allclose(oracle.softmax(np.array(k["softmax_shift"]["x"], np.float32)),
                       oracle.softmax(np.array(k["softmax_shift"]["same_as"], np.float32)), atol=d)
    sw = k["swiglu"]
    assert np.allclose(oracle.swiglu(np.array(sw["gate"], np.float32), np.array(sw["up"], np.float32)),
                       sw["expected"], atol=d)
    for key in ("rope", "rope_pos0"):
        r = k[key]
        out = oracle.rope(np.array(r["x"], np.float32), r["n_heads"], r["head_dim"], r["pos"], r["base"])
        assert np.allclose(out, r["expected"], atol=d)


def test_rope_is_a_rotation(oracle):
    x = oracle.normal(51, 8 * 128)
    y = oracle.rope(x, 8, 128, 1234, 500000.0)
    # Each (i, i+half) pair keeps its norm.
    xr, yr = x.reshape(8, 2, 64), y.reshape(8, 2, 64)
    assert np.allclose(np.hypot(xr[:, 0], xr[:, 1]), np.hypot(yr[:, 0], yr[:, 1]), rtol=1e-5)


def test_gated_activation_closed_forms(oracle):
    """SiLU(0) = 0, SiLU above 20 and GELU above 10 are the identity, below
    the low cut-offs 0, non-finite products 0."""
    g = np.array([0.0, 25.0, -25.0, 12.0, -12.0, 1.0], np.float32)
    u = np.array([3.0, 2.0, 5.0, 1.0, 1.0, np.inf], np.float32)
    s = oracle.gated_activation(g, u, 1)
    np.testing.assert_array_equal(s[:3], [0.0, 50.0, 0.0])
    assert s[5] == 0.0
    e = oracle.gated_activation(g, u, 2)
    np.testing.assert_array_equal(e[3:5], [12.0, 0.0])
    assert abs(oracle.gated_activation(np.float32([1.0]), np.float32([1.0]), 0)[0] - 1 / (1 + np.exp(-1))) < 1e-7


def test_gelu_against_erf_form_and_its_constant(oracle):
    """GELU (kind 2) is the tanh form of x * Phi(x). Against the erf form
    0.5 x (1 + erf(x / sqrt 2)) it stays within the tanh form's known largest
    deviation (about 4.73e-4 absolute, near |x| = 2.70; bound 5e-4); a
    dropped cubic term or a wrong inner constant misses by about 0.03. And it
    equals the tanh form rebuilt here from sqrt(2 / pi) and 0.044715 to fp32
    rounding."""
    import math
    x = np.linspace(-12.0, 12.0, 48001).astype(np.float32)
    got = oracle.gated_activation(x, np.ones_like(x), 2).astype(np.float64)
    xd = x.astype(np.float64)
    erf_form = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xd])
    assert np.max(np.abs(got - erf_form)) <= 5e-4
    k = math.sqrt(2.0 / math.pi)
    tanh_form = 0.5 * xd * (1.0 + np.tanh(k * (xd + 0.044715 * xd ** 3)))
    assert np.max(np.abs(got - tanh_form) / np.maximum(1.0, np.abs(tanh_form))) <= 2e-7
    # The gate times `up`, not the activation alone.
    u = np.linspace(-3.0, 3.0, x.size).astype(np.float32)
    np.testing.assert_allclose(oracle.gated_activation(x, u, 2), (tanh_form * u).astype(np.float32), rtol=2e-6,
                               atol=1e-7)
