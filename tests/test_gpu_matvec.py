"""GPU parity for the dequant-fused matvec / small-M GEMM (NF4, GGUF Q4_0 and
Q8_0, fp16 rows) against the oracle on identical seeded inputs. Tolerance:
relative L2 <= 1e-3 (fp32 outputs), the bar BASELINE.json sets."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
# Per token row, NF4 on the matrix cores (fp16-rounded activations, exact levels).
NF4_MFMA_ROW_TOL = 3e-4

# (N, K): square, gate/up (14336x4096) and down (4096x14336) Llama-3-8B shapes,
# plus small and ragged shapes.
SHAPES = [(64, 128), (96, 2080), (4096, 4096), (14336, 4096), (4096, 14336)]


def _nf4_case(oracle, n, k, group=64, seed=1):
    w = oracle.normal(seed * 7919 + n + k, n * k, 0.0, 0.02)
    codes, absmax = oracle.nf4_quantize(w, group)
    return codes, absmax


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_nf4_matvec(rocm, dev, oracle, n, k, m):
    if m > 4 and n * k > 4096 * 4096 and m != 64:
        pytest.skip("M=16 at the MLP shapes runs in test_nf4_mfma_small_m (14336x4096 and 4096x14336)")
    codes, absmax = _nf4_case(oracle, n, k)
    x = oracle.normal(11 + m, m * k)
    y_ref = oracle.nf4_matvec(codes, absmax, x, n, k, 64)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
    assert rel_l2(dev.get(y), y_ref) <= TOL


@pytest.mark.parametrize("group", [32, 128, 6])
def test_nf4_other_block_sizes(rocm, dev, oracle, group):
    n, k = 48, 384
    codes, absmax = _nf4_case(oracle, n, k, group)
    x = oracle.normal(5, k)
    y_ref = oracle.nf4_matvec(codes, absmax, x, n, k, group)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    y = dev.empty(n)
    rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, group)
    assert rel_l2(dev.get(y), y_ref) <= TOL


def test_nf4_ragged_k_uses_generic_path(rocm, dev, oracle):
    n, k = 33, 202                                         # K not a multiple of 32, odd row count
    codes, absmax = _nf4_case(oracle, n, k, 64)
    x = oracle.normal(8, 2 * k)
    y_ref = oracle.nf4_matvec(codes, absmax, x, n, k, 64)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    y = dev.empty(2 * n)
    rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, 2)
    assert rel_l2(dev.get(y), y_ref) <= TOL


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("n,k", [(64, 128), (7, 160), (4096, 4096), (14336, 4096)])
@pytest.mark.parametrize("m", [1, 8, 16])
def test_gguf_matvec(rocm, dev, oracle, qtype, n, k, m):
    if m == 16 and n == 14336:
        pytest.skip("a 32-token-accumulator variant of the Q4_0/Q8_0 matrix-core kernel (since removed) faulted "
                    "the GPU on this shape; its cause was not found, and these formats now run passes of 8 tokens")
    qt, ot = {"q4_0": (rocm.TYPE_Q4_0, oracle.QTYPE_Q4_0), "q8_0": (rocm.TYPE_Q8_0, oracle.QTYPE_Q8_0)}[qtype]
    w = oracle.normal(31 + n + k, n * k, 0.0, 0.02)
    enc = oracle.quantize(ot, w)
    x = oracle.normal(37 + m, m * k)
    y_ref = oracle.q_matvec(ot, enc, x, n, k)
    wd, xd = dev.put(enc), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
    assert rel_l2(dev.get(y), y_ref) <= TOL


# GGUF Q4_0 / Q8_0 small-M GEMM on the matrix cores (2 <= M <= 8 per pass,
# K % 512 == 0): M = 2..8 in one pass, 9..32 in several, 33 (four passes and
# a last batch-1 row), ragged N, one and several K-slices, workgroups of one,
# two and (28672 rows, Q4_0) four row tiles, the Llama shapes, and ragged N
# over K = 8192 on the register-resident kernel (several K slices, a last
# partial row tile, 8 and 8 + 5 tokens).
@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
@pytest.mark.parametrize("n,k,m", [(300, 1024, 2), (300, 1024, 3), (257, 2048, 8), (300, 1024, 9), (77, 512, 31),
                                   (300, 1536, 32), (300, 1024, 33), (4096, 14336, 8), (14336, 4096, 8),
                                   (14336, 4096, 32), (1000, 4096, 5), (28672, 4096, 8), (12345, 8192, 8),
                                   (12345, 8192, 13)])
def test_gguf_mfma_small_m(rocm, dev, oracle, qtype, n, k, m):
    qt, ot = {"q4_0": (rocm.TYPE_Q4_0, oracle.QTYPE_Q4_0), "q8_0": (rocm.TYPE_Q8_0, oracle.QTYPE_Q8_0)}[qtype]
    w = oracle.normal(53 + n + k, n * k, 0.0, 0.02)
    enc = oracle.quantize(ot, w)
    x = oracle.normal(59 + m, m * k)
    y_ref = oracle.q_matvec(ot, enc, x, n, k).ravel()
    wd, xd = dev.put(enc), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
    got = dev.get(y)
    assert rel_l2(got, y_ref) <= TOL
    for i in range(m):
        assert rel_l2(got[i * n:(i + 1) * n], y_ref[i * n:(i + 1) * n]) <= TOL, i


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0", "q4_k", "q6_k"])
def test_gguf_mfma_is_deterministic(rocm, dev, oracle, qtype):
    """The K-quant matrix-core GEMM twice over 8 K slices gives the same bits
    (the slices' partials are summed in slice order, no float atomics)."""
    n, k = 4096, 4096
    m = 8 if qtype in ("q4_0", "q8_0") else 32
    qt, ot = {"q4_0": (rocm.TYPE_Q4_0, oracle.QTYPE_Q4_0), "q8_0": (rocm.TYPE_Q8_0, oracle.QTYPE_Q8_0),
              "q4_k": (rocm.TYPE_Q4_K, oracle.QTYPE_Q4_K), "q6_k": (rocm.TYPE_Q6_K, oracle.QTYPE_Q6_K)}[qtype]
    if qtype in ("q4_0", "q8_0"):
        enc = oracle.quantize(ot, oracle.normal(71, n * k, 0.0, 0.02))
    else:   # no K-quant encoder: random super-blocks (as the concurrency test)
        enc = oracle.random_k_blocks(ot, n * k // 256, 71, scale=0.5 / np.sqrt(k) / (200 if qtype == "q4_k" else 1000))
    x = oracle.normal(73, m * k)
    wd, xd = dev.put(enc), dev.put(x)
    outs = []
    for _ in range(2):
        y = dev.empty(m * n)
        rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
        outs.append(dev.get(y))
    assert np.array_equal(outs[0], outs[1])
    assert rel_l2(outs[0], oracle.q_matvec(ot, enc, x, n, k).ravel()) <= TOL


# NF4 small-M GEMM on the matrix cores (passes of up to 64 tokens; M = 2..4
# with K % 2048 == 0 take the fp32 rows kernel): M across the 16-token tile
# and pass boundaries (31, 32, 33, 40, 64, 65, 100, 129), ragged N, the Llama
# MLP shapes, one K slice per workgroup and several (partials summed in slice
# order by a second kernel). K % 1024 == 0 runs nf4_gemm_kernel: activations
# rounded to fp16 (to nearest), levels exact (fp16 level + fp16 residual),
# fp32 accumulation, so a token row is within the activations' rounding of
# the fp32 oracle: ~2e-4 relative L2 (measured <= 2.3e-4; bound here 3e-4,
# inside the 1e-3 contract); other K (512, 1536) run the fp32-accurate
# nf4_mm_kernel. Every token row is checked on its own, so one wrong token
# tile cannot hide in the total.
@pytest.mark.parametrize("n,k,m", [(300, 1024, 2), (300, 1024, 3), (257, 2048, 8), (300, 1024, 31), (300, 1024, 32),
                                   (300, 1024, 33), (129, 512, 64), (300, 1024, 65), (77, 1536, 100),
                                   (14336, 4096, 16), (4096, 14336, 16), (4096, 14336, 64), (1000, 4096, 5),
                                   (300, 6144, 17),
                                   (8200, 4096, 32), (14336, 4096, 33), (257, 2048, 2), (14336, 4096, 64),
                                   (6144, 4096, 40), (300, 1024, 129)])
def test_nf4_mfma_small_m(rocm, dev, oracle, n, k, m):
    codes, absmax = _nf4_case(oracle, n, k, seed=3)
    x = oracle.normal(71 + m, m * k)
    y_ref = oracle.nf4_matvec(codes, absmax, x, n, k, 64).ravel()
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
    got = dev.get(y)
    assert rel_l2(got, y_ref) <= TOL
    for i in range(m):
        assert rel_l2(got[i * n:(i + 1) * n], y_ref[i * n:(i + 1) * n]) <= NF4_MFMA_ROW_TOL, i


@pytest.mark.parametrize("n,k,m", [(14336, 4096, 16), (4096, 14336, 32), (6144, 4096, 7), (14336, 4096, 64)])
def test_nf4_mfma_is_deterministic(rocm, dev, oracle, n, k, m):
    """The same GEMM twice gives the same bits (K slices are summed in a
    fixed order, no float atomics)."""
    codes, absmax = _nf4_case(oracle, n, k, seed=9)
    x = oracle.normal(91 + m, m * k)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    outs = []
    for _ in range(2):
        y = dev.empty(m * n)
        rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
        outs.append(dev.get(y))
    assert np.array_equal(outs[0], outs[1])
    y_ref = np.asarray(oracle.nf4_matvec(codes, absmax, x, n, k, 64)).reshape(m, n)
    for i in range(m):
        assert rel_l2(outs[0][i * n:(i + 1) * n], y_ref[i]) <= NF4_MFMA_ROW_TOL, i


# Batch-1 rows kernels (K % 2048 == 0): every K-chunk count S = K/2048 from 1
# to 8 (S = 3, 5, 6, 7 leave helper waves in the workgroup), row counts that
# do not fill the last workgroup, and the Llama down shape for the GGUF types.
ROWS_SHAPES = [(1, 2048), (100, 2048), (333, 6144), (77, 10240), (58, 12288), (129, 14336), (130, 16384),
               (4096, 14336)]


@pytest.mark.parametrize("fmt", ["nf4", "q4_0", "q8_0"])
@pytest.mark.parametrize("n,k", ROWS_SHAPES)
def test_batch1_rows_kernels(rocm, dev, oracle, fmt, n, k):
    w = oracle.normal(53 + n + k, n * k, 0.0, 0.02)
    x = oracle.normal(59 + k, k)
    y = dev.empty(n)
    if fmt == "nf4":
        codes, absmax = oracle.nf4_quantize(w, 64)
        y_ref = oracle.nf4_matvec(codes, absmax, x, n, k, 64)
        c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
        rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64)
    else:
        ot = oracle.QTYPE_Q4_0 if fmt == "q4_0" else oracle.QTYPE_Q8_0
        enc = oracle.quantize(ot, w)
        y_ref = oracle.q_matvec(ot, enc, x, n, k)
        wd, xd = dev.put(enc), dev.put(x)
        fn = "aljabr_rocm_matvec_tb_q4_0" if fmt == "q4_0" else "aljabr_rocm_matvec_tb_q8_0"
        rocm.call(fn, dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n)
    assert rel_l2(dev.get(y), y_ref) <= TOL


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_gguf_reference_known_rows(rocm, dev, oracle, qtype):
    import json, os
    kats = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
    k = kats["q4_0_rows" if qtype == "q4_0" else "q8_0_rows"]
    entry = "aljabr_rocm_matvec_tb_q4_0" if qtype == "q4_0" else "aljabr_rocm_matvec_tb_q8_0"
    wd = dev.put(np.array(k["blocks"], np.uint8))
    xd = dev.put(np.ones(32, np.float32))
    y = dev.empty(2)
    rocm.call(entry, dev.ptr(y), dev.ptr(xd), dev.ptr(wd), 32, 2)
    assert list(dev.get(y)) == k["dot_ones"]


@pytest.mark.parametrize("n,k,m", [(50, 136, 1), (4096, 4096, 1), (128256 // 8, 4096, 2), (300, 4096, 32)])
def test_f16_rows(rocm, dev, oracle, n, k, m):
    w = oracle.normal(41 + n, n * k).astype(np.float16).view(np.uint16)
    x = oracle.normal(43, m * k)
    y_ref = oracle.f16_matvec(w, x, n, k)
    wd, xd = dev.put(w), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, rocm.TYPE_F16, m)
    assert rel_l2(dev.get(y), y_ref) <= TOL


@pytest.mark.parametrize("n,k,m", [(1000, 512, 3), (4096 + 17, 1024, 32), (777, 2048, 33), (2048, 4096, 40),
                                   (128256 // 8, 4096, 32), (100, 4096, 2)])
def test_f16_mfma_small_m(rocm, dev, oracle, n, k, m):
    """fp16 rows with M >= 2 on the matrix cores (activations rounded to fp16,
    fp32 accumulation): every token row within the matvec tolerance, ragged
    N tiles and M above one 32-row pass included."""
    w = oracle.normal(51 + n, n * k).astype(np.float16).view(np.uint16)
    x = oracle.normal(53 + m, m * k)
    y_ref = np.asarray(oracle.f16_matvec(w, x, n, k)).ravel().reshape(m, n)
    wd, xd = dev.put(w), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, rocm.TYPE_F16, m)
    got = dev.get(y).reshape(m, n)
    for i in range(m):
        assert rel_l2(got[i], y_ref[i]) <= TOL, i


def test_batched_equals_repeated_single_rows(rocm, dev, oracle):
    """M-batched output equals M independent matvecs (the invariant the Metal
    batch test asserts, MetalTripleBatchCorrectnessTest.java:44-100)."""
    n, k, m = 512, 1024, 5
    codes, absmax = _nf4_case(oracle, n, k)
    x = oracle.normal(99, m * k)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    yb = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(yb), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
    batched = dev.get(yb).reshape(m, n)
    for i in range(m):
        xi = dev.put(x[i * k:(i + 1) * k])
        yi = dev.empty(n)
        rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(yi), dev.ptr(xi), dev.ptr(c), dev.ptr(a), k, n, 64)
        assert rel_l2(batched[i], dev.get(yi)) <= 2e-3


def test_matvec_argument_errors(rocm, dev):
    y = dev.empty(64)
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_matvec_tb_q4_0", dev.ptr(y), dev.ptr(y), dev.ptr(y), 48, 1)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:                 # Q5_K: a GGUF type without a kernel here
        rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(y), dev.ptr(y), 256, 1, 13, 1)
    assert e.value.status == rocm.ERR_UNSUPPORTED
    with pytest.raises(rocm.RocmError) as e:                 # Q4_K rows must be whole super-blocks
        rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(y), dev.ptr(y), 32, 1, 12, 1)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y), 64, 1, 7)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT


# Token-pass loops must cover exactly M rows: C rows at and past M keep a
# sentinel and every row below M equals the oracle. M = 2..7 leave a short last
# Q4_0/Q8_0 pass (8 tokens per pass), 10 a two-token pass, 31 and 33 a last
# pass of 7 and a single trailing token, 47 a second NF4 token tile of 15
# rows, across every batched row format.
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "q4_k", "q6_k", "nf4", "f16"])
@pytest.mark.parametrize("m", [2, 3, 5, 10, 31, 33, 47])
def test_batched_passes_stay_in_bounds(rocm, dev, oracle, fmt, m):
    n, k, pad = 320, 1024, 3
    w = oracle.normal(101 + m, n * k, 0.0, 0.02)
    x = oracle.normal(103 + m, (m + pad) * k)
    if fmt == "nf4":
        codes, absmax = oracle.nf4_quantize(w, 64)
        y_ref = np.asarray(oracle.nf4_matvec(codes, absmax, x[:m * k], n, k, 64)).ravel()
    elif fmt == "f16":
        enc = w.astype(np.float16).view(np.uint16)
        y_ref = np.asarray(oracle.f16_matvec(enc, x[:m * k], n, k)).ravel()
    else:
        ot = {"q4_0": oracle.QTYPE_Q4_0, "q8_0": oracle.QTYPE_Q8_0, "q4_k": oracle.QTYPE_Q4_K,
              "q6_k": oracle.QTYPE_Q6_K}[fmt]
        if fmt in ("q4_k", "q6_k"):
            enc = oracle.random_k_blocks(ot, n * k // 256, 107 + m)
        else:
            enc = oracle.quantize(ot, w)
        y_ref = np.asarray(oracle.q_matvec(ot, enc, x[:m * k], n, k)).ravel()
    sentinel = np.full((m + pad) * n, -12345.5, np.float32)
    y, xd = dev.put(sentinel), dev.put(x)
    if fmt == "nf4":
        c, a = dev.put(codes), dev.put(absmax)
        rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
    else:
        qt = {"q4_0": rocm.TYPE_Q4_0, "q8_0": rocm.TYPE_Q8_0, "q4_k": rocm.TYPE_Q4_K, "q6_k": rocm.TYPE_Q6_K,
              "f16": rocm.TYPE_F16}[fmt]
        wd = dev.put(enc)
        rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
    got = dev.get(y)
    assert np.all(got[m * n:] == np.float32(-12345.5)), "rows past M were written"
    for i in range(m):
        assert rel_l2(got[i * n:(i + 1) * n], y_ref[i * n:(i + 1) * n]) <= TOL, i


# NF4 with M = 2..4 tokens runs the batch-1 rows kernel with every lookup
# feeding each token (fp32 throughout): every token row within 1e-5 of the
# oracle, at the Llama MLP shapes, one K chunk, seven K chunks (one helper
# wave) and a row count that does not fill the last workgroup.
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336), (300, 2048), (77, 10240)])
@pytest.mark.parametrize("m", [2, 3, 4])
def test_nf4_small_m_fp32_rows(rocm, dev, oracle, n, k, m):
    codes, absmax = _nf4_case(oracle, n, k, seed=5)
    x = oracle.normal(81 + m, m * k)
    y_ref = np.asarray(oracle.nf4_matvec(codes, absmax, x, n, k, 64)).reshape(m, n)
    c, a, xd = dev.put(codes), dev.put(absmax), dev.put(x)
    y = dev.put(np.full((m + 1) * n, -7.5, np.float32))
    rocm.call("aljabr_rocm_matvec_tb_batch_nf4", dev.ptr(y), dev.ptr(xd), dev.ptr(c), dev.ptr(a), k, n, 64, m)
    got = dev.get(y)
    assert np.all(got[m * n:] == np.float32(-7.5))
    got = got[:m * n].reshape(m, n)
    for i in range(m):
        assert rel_l2(got[i], y_ref[i]) <= 1e-5, i
