"""Write ``reference_kats.json``: the known-answer data held by the reference's
own JUnit tests for this hot path, transcribed as data (inputs and the
expected outputs those tests assert). Nothing here runs reference code; each
entry cites the test file:line it comes from. Paths are relative to the
andalus-ai/aljabr tree:

  GRTT = engine/gguf/aljabr-gguf-core/src/test/java/tech/kayys/aljabr/gguf/runtime
  CPUT = backend/cpu/aljabr-backend-cpu/src/test/java/tech/kayys/aljabr/backend/cpu
  GJBT = engine/gguf/aljabr-gguf-java/src/test/java/tech/kayys/aljabr/gguf/javabackend

Run ``python tests/golden/make_reference_kats.py`` to regenerate.
"""
from __future__ import annotations

import json
import math
import os

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
NEG_INF = "-inf"
POS_INF = "inf"
NAN = "nan"


def q4_block(scale_bits: int, packed: int) -> list[int]:
    """GRTT/GgufQ32Q4Fx.java:17-20,57-61: f16 scale then 16 copies of one byte."""
    return [scale_bits & 0xFF, scale_bits >> 8] + [packed & 0xFF] * 16


def q8_block(scale_bits: int, quant: int) -> list[int]:
    """GRTT/GgufQ8Fx.java:19-24: f16 scale then 32 copies of one byte."""
    return [scale_bits & 0xFF, scale_bits >> 8] + [quant & 0xFF] * 32


def q8_pattern(seed: int, index: int) -> int:
    """GRTT/GgufQ8RawTest.java:399-401: (byte)(seed + 41*index)."""
    return (seed + 41 * index) & 0xFF


def main() -> None:
    kats = {}

    # GRTT/GgufQ32Test.java:17-42: two Q4_0 rows, scale 1.0, bytes 0x98 / 0xA9.
    kats["q4_0_rows"] = {
        "source": "GRTT/GgufQ32Test.java:17-42",
        "blocks": q4_block(0x3C00, 0x98) + q4_block(0x3C00, 0xA9),
        "columns": 32,
        "rows": 2,
        "row0": [0.0] * 16 + [1.0] * 16,
        "dot_ones": [16.0, 48.0],
    }

    # GRTT/GgufQ32RawTest.java:72-105,221-235: five Q4_0 blocks, patterned vector.
    kats["q4_0_raw_pattern"] = {
        "source": "GRTT/GgufQ32RawTest.java:72-105,221-235",
        "half_scales": [0x3C00, 0x4000, 0xBC00, 0x3800, 0x4200],
        "scales": [1.0, 2.0, -1.0, 0.5, 3.0],
        "packed": [0x21, 0x43, 0x65, 0x87, 0xA9],
        "vector": [(i % 23 - 11) * 0.0625 for i in range(5 * 32)],
        "tolerance": 1.0e-3,
    }

    # GRTT/GgufNibFx.java:13-25 with GRTT/GgufQ32Q4Fx.java:22-25,40-47:
    # byte i = low(i) | high(i) << 4, low(i) = i, high(i) = 15 - i; the expected
    # row for Q4_0 (zero point 8, bias 0) is low(i)-8 then high(i)-8, times d.
    kats["q4_0_lane_order"] = {
        "source": "GRTT/GgufNibFx.java:13-25; GRTT/GgufQ32Q4Fx.java:22-25,40-47",
        "scale_bits": 0x3C00,
        "codes": [(i & 0x0F) | ((15 - i) << 4) for i in range(16)],
        "expected_row": [float(i - 8) for i in range(16)] + [float(15 - i - 8) for i in range(16)],
    }

    # GRTT/GgufQ8Test.java:22-40: Q8_0 rows of 1s and 2s, scale 1.0, dot with ones.
    kats["q8_0_rows"] = {
        "source": "GRTT/GgufQ8Test.java:22-40",
        "blocks": q8_block(0x3C00, 1) + q8_block(0x3C00, 2),
        "columns": 32,
        "rows": 2,
        "dot_ones": [32.0, 64.0],
    }

    # GRTT/GgufQ8RawTest.java:238-261,380-401: five patterned Q8_0 blocks, vector
    # (i % 19 - 9) * 0.0625 read from offset 5, tolerance 1e-3.
    seeds = [11, 29, 47, 83, 109]
    half = [0x3C00, 0x4000, 0xBC00, 0x4200, 0x3800]
    blocks = []
    for s, h in zip(seeds, half):
        blocks += [h & 0xFF, h >> 8] + [q8_pattern(s, i) for i in range(32)]
    vec = [(i % 19 - 9) * 0.0625 for i in range(5 * 32 + 5)]
    kats["q8_0_raw_pattern"] = {
        "source": "GRTT/GgufQ8RawTest.java:238-261,380-401",
        "blocks": blocks,
        "scales": [1.0, 2.0, -1.0, 3.0, 0.5],
        "seeds": seeds,
        "vector": vec,
        "vector_offset": 5,
        "tolerance": 1.0e-3,
    }

    # ---- K-quants. Block builders of GRTT/GgufQ4Fx.java:11-58,
    # GRTT/GgufQ4CalcFx.java:11-49, GRTT/GgufQ6Fx.java:11-52 and
    # GRTT/GgufQ6LaneFx.java:11-61, written out as bytes; the expected values
    # are the ones those tests assert (or the fixture's own expected rows).
    def q4k_header(d_bits, dmin_bits, scales):
        return [d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8] + list(scales)

    q4k_simple_scales = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    q4k_mins_scales = [1, 1, 1, 1, 2, 2, 2, 2, 0x21, 0x21, 0x21, 0x21]
    simple = q4k_header(0x3C00, 0, q4k_simple_scales) + [0x21] * 128
    with_mins = q4k_header(0x3C00, 0x3800, q4k_mins_scales) + [0x21] * 128
    nan_dmin = q4k_header(0x3C00, 0x7E00, q4k_simple_scales) + [0x21] * 128
    kats["q4_k_rows"] = {
        "source": "GRTT/GgufQ4KPrepTest.java:22-40,67-84; GRTT/GgufQ4KMixTest.java:21-43; "
                  "GRTT/GgufKZeroMinTest.java:20-52",
        "simple": simple,               # d=1, dMin=0, every scale 1, no mins: dot(ones) = 1*128 + 2*128
        "with_mins": with_mins,         # d=1, dMin=0.5, scale 1, min 2 (-1.0): dot(ones) = 0*128 + 1*128
        "nan_dmin_zero_mins": nan_dmin, # dMin NaN with every min code 0: no min term, as simple
        "dot_ones": {"simple": 384.0, "with_mins": 128.0, "nan_dmin_zero_mins": 384.0},
    }

    lane_q = [(i & 0x0F) | ((15 - (i & 0x0F)) << 4) for i in range(128)]
    def q4k_lane_row(has_mins):
        row = [0.0] * 256
        for sb in range(0, 256, 64):
            qb = (sb // 64) * 32
            for i in range(32):
                low = (qb + i) & 0x0F
                row[sb + i] = float(low - 1 if has_mins else low)
                row[sb + 32 + i] = float((15 - low) - 1 if has_mins else 15 - low)
        return row
    kats["q4_k_lane_order"] = {
        "source": "GRTT/GgufQ4Fx.java:37-58; GRTT/GgufQ4CalcFx.java:11-49",
        "no_mins": {"block": q4k_header(0x3C00, 0, q4k_simple_scales) + lane_q,
                    "expected_row": q4k_lane_row(False)},
        "mins": {"block": q4k_header(0x3C00, 0x3800, q4k_mins_scales) + lane_q,
                 "expected_row": q4k_lane_row(True)},
    }

    def q6k_block(low_packed, high_packed, scale):
        return [low_packed] * 128 + [high_packed] * 64 + [scale & 0xFF] * 16 + [0x00, 0x3C]
    kats["q6_k_rows"] = {
        "source": "GRTT/GgufQ6Fx.java:11-27; GRTT/GgufQ6KPrepTest.java:19-36",
        "ones": q6k_block(0x11, 0xAA, 1),     # q6 = 1 | 2<<4 = 33 -> 1.0 everywhere
        "twos": q6k_block(0x22, 0xAA, 1),     # q6 = 34 -> 2.0 everywhere: dot(ones) = 512
        "dot_ones": {"ones": 256.0, "twos": 512.0},
    }

    q6_low = [(i & 0x0F) | ((15 - (i & 0x0F)) << 4) for i in range(128)]
    q6_high = [(i * 53 + 0xA7) & 0xFF for i in range(64)]
    q6_row = [0.0] * 256
    for sb in range(0, 256, 128):
        lb, hb = (sb // 128) * 64, (sb // 128) * 32
        for i in range(32):
            la, lbv, hbits = q6_low[lb + i], q6_low[lb + 32 + i], q6_high[hb + i]
            q6_row[sb + i] = float(((la & 0x0F) | ((hbits & 3) << 4)) - 32)
            q6_row[sb + 32 + i] = float(((lbv & 0x0F) | (((hbits >> 2) & 3) << 4)) - 32)
            q6_row[sb + 64 + i] = float(((la >> 4) | (((hbits >> 4) & 3) << 4)) - 32)
            q6_row[sb + 96 + i] = float(((lbv >> 4) | (((hbits >> 6) & 3) << 4)) - 32)
    kats["q6_k_lane_order"] = {
        "source": "GRTT/GgufQ6Fx.java:29-52; GRTT/GgufQ6LaneFx.java:11-61",
        "block": q6_low + q6_high + [1] * 16 + [0x00, 0x3C],
        "expected_row": q6_row,
    }

    # CPUT/CpuBatchedAttentionTest.java (all through CpuBackend.attention ->
    # attentionGqa with Hq == Hkv): shapes [B,H,S,D].
    att = []
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:13-31",
        "q_shape": [1, 2, 2, 2], "k_shape": [1, 2, 3, 2],
        "q": [0.0] * 8, "k": [0.0] * 12,
        "v": [1, 3, 3, 5, 5, 7, 2, 4, 4, 6, 6, 8],
        "mask": None, "causal": False,
        "expected": [3, 5, 3, 5, 4, 6, 4, 6], "tolerance": 1e-5,
    })
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:49-68 (mask)",
        "q_shape": [1, 1, 2, 1], "k_shape": [1, 1, 2, 1],
        "q": [0.0, 0.0], "k": [0.0, 0.0], "v": [2.0, 8.0],
        "mask": [0.0, NEG_INF, 0.0, NEG_INF], "causal": False,
        "expected": [2.0, 2.0], "tolerance": 1e-6,
    })
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:49-68 (causal)",
        "q_shape": [1, 1, 2, 1], "k_shape": [1, 1, 2, 1],
        "q": [0.0, 0.0], "k": [0.0, 0.0], "v": [2.0, 8.0],
        "mask": None, "causal": True,
        "expected": [2.0, 5.0], "tolerance": 1e-6,
    })
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:70-87",
        "q_shape": [1, 1, 2, 1], "k_shape": [1, 1, 4, 1],
        "q": [0.0, 0.0], "k": [0.0] * 4, "v": [1.0, 3.0, 5.0, 7.0],
        "mask": None, "causal": True,
        "expected": [3.0, 4.0], "tolerance": 1e-6,
    })
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:88-104",
        "q_shape": [1, 1, 3, 1], "k_shape": [1, 1, 2, 1],
        "q": [0.0] * 3, "k": [0.0] * 2, "v": [2.0, 8.0],
        "mask": None, "causal": True,
        "expected": [0.0, 2.0, 5.0], "tolerance": 1e-6,
    })
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:161-176",
        "q_shape": [1, 1, 1, 1], "k_shape": [1, 1, 2, 1],
        "q": [0.0], "k": [0.0, 0.0], "v": [2.0, 8.0],
        "mask": [NEG_INF, NEG_INF], "causal": False,
        "expected": [0.0], "tolerance": 1e-6,
    })
    logits = [0.0, 2.0, 1.0, 3.0, -1.0]
    values = [1.0, 2.0, 3.0, 4.0, 5.0]
    mx = max(logits)
    den = sum(math.exp(l - mx) for l in logits)
    wsum = sum(math.exp(l - mx) * v for l, v in zip(logits, values))
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:178-206 (expected computed as the test does)",
        "q_shape": [1, 1, 1, 1], "k_shape": [1, 1, 5, 1],
        "q": [1.0], "k": logits, "v": values,
        "mask": None, "causal": False,
        "expected": [wsum / den], "tolerance": 1e-6,
    })
    qv = [0.7, -0.3]
    kv = [0.2, 0.8, -0.4, 0.1, 0.9, -0.2, 0.3, 0.5, -0.7, -0.6]
    vv = [1.0, 2.0, 3.0, -1.0, -2.0, 4.0, 0.5, 0.25, 5.0, -3.0]
    lg = [(qv[0] * kv[2 * i] + qv[1] * kv[2 * i + 1]) / math.sqrt(2.0) for i in range(5)]
    m2 = max(lg)
    p = [math.exp(x - m2) for x in lg]
    e0 = sum(pi * vv[2 * i] for i, pi in enumerate(p)) / sum(p)
    e1 = sum(pi * vv[2 * i + 1] for i, pi in enumerate(p)) / sum(p)
    att.append({
        "source": "CPUT/CpuBatchedAttentionTest.java:208-258 (expected computed as the test does)",
        "q_shape": [1, 1, 1, 2], "k_shape": [1, 1, 5, 2],
        "q": qv, "k": kv, "v": vv,
        "mask": None, "causal": False,
        "expected": [e0, e1], "tolerance": 1e-5,
    })
    # CPUT/CpuBackendStorageTest.java:1239-1274: GQA, two query heads on one
    # KV head; the strided views resolve to these logical values.
    att.append({
        "source": "CPUT/CpuBackendStorageTest.java:1239-1274",
        "q_shape": [1, 2, 2, 2], "k_shape": [1, 1, 2, 2],
        "q": [0.0] * 8, "k": [1.0, 3.0, 2.0, 4.0], "v": [2.0, 3.0, 4.0, 5.0],
        "mask": None, "causal": False,
        "expected": [3.0, 4.0, 3.0, 4.0, 3.0, 4.0, 3.0, 4.0], "tolerance": 1e-6,
    })
    kats["attention"] = att
    kats["attention_rejects"] = [
        {"source": "CPUT/CpuBatchedAttentionTest.java:106-124", "mask": [0.0, NAN, 0.0, 0.0], "causal": True},
        {"source": "CPUT/CpuBatchedAttentionTest.java:126-141", "mask": [0.0, NAN, 0.0, 0.0], "causal": False},
        {"source": "CPUT/CpuBatchedAttentionTest.java:143-159", "mask": [0.0, 0.0, POS_INF, 0.0], "causal": False},
    ]

    # GJBT/GGUFVectorOpsTest.java:60-150
    kats["vector_ops"] = {
        "source": "GJBT/GGUFVectorOpsTest.java:60-150",
        "delta": 1e-4,
        "rmsnorm": [
            {"x": [1, 2, 3, 4], "w": [1, 1, 1, 1], "eps": 1e-5,
             "expected": [0.36514813, 0.73029625, 1.0954444, 1.4605925]},
            {"x": [2, -1, 0.5, 3], "w": [1.0, 2.0, 0.5, 1.5], "eps": 1e-5,
             "expected": [1.0596244, -1.0596244, 0.13245305, 2.384155]},
        ],
        "softmax": {"x": [1, 2, 3], "expected": [0.09003057, 0.24472847, 0.66524096]},
        "softmax_shift": {"x": [10000, 10001, 10002], "same_as": [1, 2, 3]},
        "swiglu": {"gate": [0, 1, -1], "up": [2, 2, 2], "expected": [0.0, 1.4621172, -0.5378828]},
        "rope": {"x": [1, 0, 1, 0], "n_heads": 1, "head_dim": 4, "pos": 1, "base": 10000.0,
                 "expected": [-0.30116868, 0.0, 1.3817733, 0.0]},
        "rope_pos0": {"x": [1, 2, 3, 4], "n_heads": 1, "head_dim": 4, "pos": 0, "base": 10000.0,
                      "expected": [1, 2, 3, 4]},
    }

    # GJBT/GgufDecodeAttentionExecutionTest.java:15-66: the decode runner's
    # attention (GgufDecodeAttentionExecution.execute over position-major
    # [position][cache_head_stride] arrays). Arguments in the order of the
    # array form: cache_head_stride, kv_heads, query_heads, head_dim,
    # sequence_length, start_position, scale. The session case (:48-66) reads
    # positions 1..2 of a one-head cache holding values 10, 20, 30; its window
    # is the same call on those three positions with start 1.
    kats["decode_attention"] = [
        {"source": "GJBT/GgufDecodeAttentionExecutionTest.java:15-29",
         "query": [0.0] * 4, "keys": [0.0] * 4, "values": [10.0, 100.0, 20.0, 200.0],
         "args": [2, 2, 4, 1, 2, 0, 1.0], "expected": [15.0, 15.0, 150.0, 150.0], "tolerance": 1e-6},
        {"source": "GJBT/GgufDecodeAttentionExecutionTest.java:31-44",
         "query": [0.0, 0.0], "keys": [0.0] * 4, "values": [10.0, 100.0, 20.0, 200.0],
         "args": [2, 2, 2, 1, 2, 1, 1.0], "expected": [20.0, 200.0], "tolerance": 1e-6},
        {"source": "GJBT/GgufDecodeAttentionExecutionTest.java:45-66",
         "query": [0.0], "keys": [0.0] * 3, "values": [10.0, 20.0, 30.0],
         "args": [1, 1, 1, 1, 3, 1, 1.0], "expected": [25.0], "tolerance": 1e-6},
    ]

    with open(OUT, "w") as f:
        json.dump(kats, f, indent=1)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
