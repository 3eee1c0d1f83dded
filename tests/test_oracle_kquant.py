"""Pins the oracle's GGUF K-quant functions (Q4_K, Q6_K; CPU only).

Known answers come from the reference's JUnit fixtures
(tests/golden/reference_kats.json: q4_k_rows, q4_k_lane_order, q6_k_rows,
q6_k_lane_order). Where they leave gaps (the high two bits of the packed
Q4_K scale/min codes, which every fixture leaves zero; distinct Q6_K scales
per 16 elements) the checks use blocks built by an independent packer written
from the GGUF format description below, so a swapped index or shift in the
oracle's unpacking fails here:

* Q4_K super-block (144 bytes): f16 d, f16 dmin, 12 bytes holding eight 6-bit
  scales sc[j] and eight 6-bit mins m[j], 128 bytes of nibbles. For j < 4,
  byte j carries sc[j] in its low 6 bits and byte j+4 carries m[j]; for j >= 4,
  byte j+4 carries sc[j] (low nibble) and m[j] (high nibble) low 4 bits, and the
  top two bits of bytes j-4 and j carry the high 2 bits of sc[j] and m[j].
  Sub-block j covers elements 32j..32j+31: element 64c+l (l < 32) is the low
  nibble of byte 32c+l, element 64c+32+l its high nibble.
  Value = d*sc[j]*q - dmin*m[j].
* Q6_K super-block (210 bytes): ql[128], qh[64], int8 scales[16], f16 d.
  Element e has scale scales[e // 16]; value = d*scale*(q6 - 32).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import rel_l2

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
Q4_K, Q6_K = 12, 14


def _u8(xs):
    return np.array(xs, dtype=np.uint8)


# ------------------------------------------------------------- known answers

def test_q4_k_fixture_rows(oracle):
    k = KATS["q4_k_rows"]
    ones = np.ones(256, np.float32)
    for name in ("simple", "with_mins", "nan_dmin_zero_mins"):
        blk = _u8(k[name])
        w = oracle.dequant(Q4_K, blk, 256)
        assert not np.isnan(w).any(), name            # a zero min code adds nothing, NaN dMin included
        assert oracle.dot_row(Q4_K, blk, ones) == k["dot_ones"][name]
        assert float(w.astype(np.float64).sum()) == k["dot_ones"][name]
    # Two rows through the matvec, as GgufQ4KMixTest reads them.
    both = np.concatenate([_u8(k["nan_dmin_zero_mins"]), _u8(k["with_mins"])])
    y = oracle.q_matvec(Q4_K, both, ones, 2, 256, nthreads=1)
    assert y.tolist() == [384.0, 128.0]


@pytest.mark.parametrize("case", ["no_mins", "mins"])
def test_q4_k_lane_order(oracle, case):
    k = KATS["q4_k_lane_order"][case]
    blk = _u8(k["block"])
    exp = np.array(k["expected_row"], np.float32)
    assert np.array_equal(oracle.dequant(Q4_K, blk, 256), exp)
    ramp = np.arange(1, 257, dtype=np.float32)
    # Integer products and partial sums below 2^24: every fp32 order is exact.
    assert oracle.dot_row(Q4_K, blk, ramp) == float(exp.astype(np.int64) @ ramp.astype(np.int64))


def test_q6_k_fixture_rows(oracle):
    k = KATS["q6_k_rows"]
    ones = np.ones(256, np.float32)
    for name, val in (("ones", 1.0), ("twos", 2.0)):
        blk = _u8(k[name])
        assert np.all(oracle.dequant(Q6_K, blk, 256) == val)
        assert oracle.dot_row(Q6_K, blk, ones) == k["dot_ones"][name]


def test_q6_k_lane_order(oracle):
    k = KATS["q6_k_lane_order"]
    blk = _u8(k["block"])
    exp = np.array(k["expected_row"], np.float32)
    assert np.array_equal(oracle.dequant(Q6_K, blk, 256), exp)
    ramp = np.arange(1, 257, dtype=np.float32)
    assert oracle.dot_row(Q6_K, blk, ramp) == float(exp.astype(np.int64) @ ramp.astype(np.int64))


# ------------------------------------------- independent packers (format text)

def pack_q4_k_scales(sc, mn):
    """12 bytes from eight 6-bit scales and mins, per the module docstring."""
    b = [0] * 12
    for j in range(8):
        if j < 4:
            b[j] |= sc[j] & 63
            b[j + 4] |= mn[j] & 63
        else:
            b[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            b[j - 4] |= (sc[j] >> 4) << 6
            b[j] |= (mn[j] >> 4) << 6
    return b


def q4_k_block(d, dmin, sc, mn, q):
    """q: 256 nibble values in element order."""
    hdr = np.array([d, dmin], np.float16).view(np.uint8).tolist()
    qs = [0] * 128
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    return _u8(hdr + pack_q4_k_scales(sc, mn) + qs)


@pytest.mark.parametrize("seed", range(6))
def test_q4_k_scale_min_codes_round_trip(oracle, seed):
    rng = np.random.default_rng(seed)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    if seed == 0:
        sc[:] = 63
        mn[:] = 63                                    # every high bit set
    mn[seed % 8] = 0                                  # one sub-block without a min
    q = rng.integers(0, 16, 256)
    d, dmin = np.float16(0.5), np.float16(0.25)
    blk = q4_k_block(d, dmin, sc.tolist(), mn.tolist(), q.tolist())
    w = oracle.dequant(Q4_K, blk, 256)
    j = np.arange(256) // 32
    exp = (np.float32(d) * sc[j].astype(np.float32)) * q.astype(np.float32) - \
        np.where(mn[j] == 0, np.float32(0), np.float32(dmin) * mn[j].astype(np.float32))
    assert np.array_equal(w, exp.astype(np.float32))


def q6_k_block(d, scales, q6):
    """q6: 256 six-bit values in element order; scales: 16 int8."""
    ql = [0] * 128
    qh = [0] * 64
    for h in range(2):
        for l in range(32):
            e = [128 * h + l + 32 * k for k in range(4)]
            ql[64 * h + l] = (q6[e[0]] & 15) | ((q6[e[2]] & 15) << 4)
            ql[64 * h + 32 + l] = (q6[e[1]] & 15) | ((q6[e[3]] & 15) << 4)
            qh[32 * h + l] = sum(((q6[e[k]] >> 4) & 3) << (2 * k) for k in range(4))
    return _u8(ql + qh + np.array(scales, np.int8).view(np.uint8).tolist()
               + np.array([d], np.float16).view(np.uint8).tolist())


@pytest.mark.parametrize("seed", range(6))
def test_q6_k_packed_round_trip(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    scales = rng.integers(-128, 128, 16)
    q6 = rng.integers(0, 64, 256)
    d = np.float16(rng.uniform(-1, 1))
    blk = q6_k_block(d, scales.tolist(), q6.tolist())
    w = oracle.dequant(Q6_K, blk, 256)
    e = np.arange(256)
    exp = (np.float32(d) * scales[e // 16].astype(np.float32)) * (q6 - 32).astype(np.float32)
    assert np.array_equal(w, exp.astype(np.float32))


# -------------------------------------------------------- dots against brute force

@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("k", [256, 768, 1024, 4096])
def test_k_dot_row_matches_float64(oracle, qtype, k):
    blocks = oracle.random_k_blocks(qtype, 3 * k // 256, seed=k + qtype)
    x = np.random.default_rng(k).standard_normal(3 * k).astype(np.float32)
    dense = oracle.dequant(qtype, blocks, 3 * k).reshape(3, k).astype(np.float64)
    bb = oracle.block_bytes(qtype) * (k // 256)
    for r in range(3):
        got = oracle.dot_row(qtype, blocks[r * bb:(r + 1) * bb], x[r * k:(r + 1) * k])
        ref = float(dense[r] @ x[r * k:(r + 1) * k].astype(np.float64))
        assert abs(got - ref) <= 1e-5 * (abs(ref) + np.abs(dense[r]).sum() * 1e-2)
    # The matvec is the dot per row, for every token row.
    xm = np.random.default_rng(k + 1).standard_normal((2, k)).astype(np.float32)
    y = oracle.q_matvec(qtype, blocks, xm, 3, k)
    exp = xm.astype(np.float64) @ dense.T
    assert rel_l2(y, exp) < 1e-6


def test_k_quant_min_term_sign(oracle):
    """A plausible mistake, adding dMin*min instead of subtracting, fails: a
    block of zero nibbles decodes to -dMin*min exactly."""
    sc = [1] * 8
    mn = [3] * 8
    blk = q4_k_block(np.float16(1.0), np.float16(0.5), sc, mn, [0] * 256)
    assert np.all(oracle.dequant(Q4_K, blk, 256) == -1.5)
    assert oracle.dot_row(Q4_K, blk, np.ones(256, np.float32)) == -384.0


def test_softcap_closed_form(oracle):
    y = np.array([0.0, 1e-3, -1e-3, 1.0, -2.0, 50.0, -1e4], np.float32)
    got = oracle.softcap(y, 30.0)
    exp = (30.0 * np.tanh(y.astype(np.float64) / 30.0)).astype(np.float32)
    assert np.allclose(got, exp, rtol=1e-6, atol=0)
    assert got[0] == 0.0 and abs(got[-1] + 30.0) < 1e-5
