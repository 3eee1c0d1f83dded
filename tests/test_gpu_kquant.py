"""GPU parity for the GGUF K-quants (Q4_K, Q6_K): bit-exact dequantization
and the matvec / small-M GEMM (relative L2 <= 1e-3 against the oracle's
restatement of GgufQ4RawDot / GgufQ6RawDot on the same seeded blocks), the
output soft cap, the reference's fixture known answers through the GPU, and
the status codes."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-3
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))
TYPES = {"q4_k": 12, "q6_k": 14}


def _blocks(oracle, qt, n, k, seed):
    return oracle.random_k_blocks(qt, n * k // 256, seed=seed)


def _special_q4k_blocks(nblocks, seed):
    """Random Q4_K blocks with the header cases the decoders must honour: dmin
    NaN (zero and non-zero min codes), dmin 0, -0, negative d, subnormal d."""
    import oracle as orc
    b = orc.random_k_blocks(12, nblocks, seed).reshape(nblocks, 144)
    hdr = [(0x3C00, 0x7E00), (0x3C00, 0x0000), (0x3C00, 0x8000), (0xBC00, 0x3800), (0x0001, 0x3400),
           (0x3C00, 0x7E00)]
    for i, (d, dm) in enumerate(hdr):
        b[i, 0:4] = [d & 0xFF, d >> 8, dm & 0xFF, dm >> 8]
    b[0, 4:16] = 0                      # NaN dmin, every min code zero: finite
    return b.ravel()


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
def test_kquant_dequant_bit_exact(rocm, dev, oracle, qtype):
    qt = TYPES[qtype]
    nb = 777
    blocks = _special_q4k_blocks(nb, 5) if qt == 12 else oracle.random_k_blocks(qt, nb, 6)
    exp = oracle.dequant(qt, blocks, nb * 256)
    src = dev.put(blocks)
    out = dev.empty(nb * 256)
    rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(src), None, nb * 256, qt, 0)
    got = dev.get(out)
    nan = np.isnan(exp)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))
    if qt == 12:
        assert not nan[:256].any()                  # NaN dmin, zero min codes: finite
        assert nan[5 * 256:6 * 256].any()           # NaN dmin, non-zero min codes: NaN there
        assert not nan[6 * 256:].any()


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
@pytest.mark.parametrize("n,k", [(1, 256), (7, 768), (64, 2048), (100, 4096), (333, 6144), (4096, 4096),
                                 (14336, 4096), (4096, 14336), (130, 16384), (3, 17408)])
@pytest.mark.parametrize("m", [1, 3, 8, 13])
def test_kquant_matvec(rocm, dev, oracle, qtype, n, k, m):
    if m > 3 and n * k > 4096 * 4096:
        pytest.skip("large shapes at m = 1, 3")
    qt = TYPES[qtype]
    blocks = _blocks(oracle, qt, n, k, seed=n + k + qt)
    x = oracle.normal(41 + m + k, m * k)
    y_ref = oracle.q_matvec(qt, blocks, x, n, k).ravel()
    wd, xd = dev.put(blocks), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
    got = dev.get(y)
    assert rel_l2(got, y_ref) <= TOL
    for i in range(m):
        assert rel_l2(got[i * n:(i + 1) * n], y_ref[i * n:(i + 1) * n]) <= TOL, i


# Matrix-core path (2 <= M <= 32 per pass, K % 512 == 0): M across the pass
# boundary (33 = 32 + a batch-1 row, 40 = 32 + 8), ragged N, the MLP shapes
# (256- and 512-element K slices; 28672 rows take four row tiles per wave in
# Q4_K; the stacked gate/up of Llama-3-8B at the full 32-token pass), ragged
# N over K = 8192 with one and two 16-token tiles (Q4_K's register-resident
# kernel), and the Q4_K header cases (NaN dmin with zero min codes, dmin 0,
# -0).
@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
@pytest.mark.parametrize("n,k,m", [(300, 512, 2), (257, 1024, 5), (300, 2048, 16), (77, 1536, 31), (129, 4096, 32),
                                   (300, 1024, 33), (100, 3072, 40), (14336, 4096, 8), (4096, 14336, 32),
                                   (28672, 4096, 8), (28672, 4096, 32), (12345, 8192, 5), (12345, 8192, 20)])
def test_kquant_mfma(rocm, dev, oracle, qtype, n, k, m):
    qt = TYPES[qtype]
    blocks = _blocks(oracle, qt, n, k, seed=3 * n + k + m)
    if qt == 12:
        special = _special_q4k_blocks(6, 17).reshape(6, 144)
        b = blocks.reshape(-1, 144)
        b[:5] = special[:5]                     # the first row's first super-blocks
    x = oracle.normal(61 + m + k, m * k)
    y_ref = oracle.q_matvec(qt, blocks, x, n, k).ravel()
    wd, xd = dev.put(blocks), dev.put(x)
    y = dev.empty(m * n)
    rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, qt, m)
    got = dev.get(y)
    assert np.isfinite(got).all()
    for i in range(m):
        assert rel_l2(got[i * n:(i + 1) * n], y_ref[i * n:(i + 1) * n]) <= TOL, i


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
@pytest.mark.parametrize("n,k", [(1, 2048), (100, 2048), (333, 6144), (77, 10240), (4096, 14336)])
def test_kquant_batch1_entry_points(rocm, dev, oracle, qtype, n, k):
    qt = TYPES[qtype]
    blocks = _blocks(oracle, qt, n, k, seed=7 * n + k)
    x = oracle.normal(3 + k, k)
    y_ref = oracle.q_matvec(qt, blocks, x, n, k)
    wd, xd = dev.put(blocks), dev.put(x)
    y = dev.empty(n)
    rocm.call(f"aljabr_rocm_matvec_tb_{qtype}", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n)
    assert rel_l2(dev.get(y), y_ref) <= TOL


@pytest.mark.parametrize("qtype", ["q4_k", "q6_k"])
@pytest.mark.parametrize("cap", [0.0, 30.0, 2.5])
def test_kquant_softcap(rocm, dev, oracle, qtype, cap):
    qt = TYPES[qtype]
    n, k = 515, 4096
    blocks = _blocks(oracle, qt, n, k, seed=91)
    x = oracle.normal(92, k, 0.0, 3.0)
    y_ref = oracle.q_matvec(qt, blocks, x, n, k)
    if cap > 0:
        y_ref = oracle.softcap(y_ref, cap)
    wd, xd = dev.put(blocks), dev.put(x)
    y = dev.empty(n)
    rocm.call(f"aljabr_rocm_matvec_tb_{qtype}_softcap", dev.ptr(y), dev.ptr(xd), dev.ptr(wd), k, n, cap)
    got = dev.get(y)
    assert rel_l2(got, y_ref) <= TOL
    if cap > 0:
        assert np.abs(got).max() <= cap


def test_kquant_fixture_answers_on_gpu(rocm, dev):
    """The reference fixtures' rows through the GPU matvec: integer-valued
    products, so the answers are exact."""
    k4, k6 = KATS["q4_k_rows"], KATS["q6_k_rows"]
    cases = [(12, k4["simple"], 384.0), (12, k4["with_mins"], 128.0), (12, k4["nan_dmin_zero_mins"], 384.0),
             (14, k6["ones"], 256.0), (14, k6["twos"], 512.0)]
    ones = dev.put(np.ones(256, np.float32))
    for qt, blk, want in cases:
        wd = dev.put(np.array(blk, np.uint8))
        y = dev.empty(1)
        rocm.call("aljabr_rocm_matvec_tb_batch", dev.ptr(y), dev.ptr(ones), dev.ptr(wd), 256, 1, qt, 1)
        assert dev.get(y)[0] == want, (qt, want)


def test_kquant_statuses(rocm, dev):
    x = dev.put(np.ones(1024, np.float32))
    w = dev.put(np.zeros(4 * 210 * 4, np.uint8))
    y = dev.empty(64)
    with pytest.raises(rocm.RocmError) as e:                 # K not whole super-blocks
        rocm.call("aljabr_rocm_matvec_tb_q4_k", dev.ptr(y), dev.ptr(x), dev.ptr(w), 320, 2)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:                 # misaligned activations
        rocm.call("aljabr_rocm_matvec_tb_q6_k", dev.ptr(y), dev.ptr(x) + 4, dev.ptr(w), 256, 2)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_dequantize", dev.ptr(y), dev.ptr(w), None, 200, 14, 0)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
