"""GPU parity for the codecs: device decoders must be bit-exact with the oracle
(the reference's decoders restated), device encoders bit-exact with the
oracle's GGUFWriter restatement. Calls go through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def _random_f16_scales(rng, n):
    """fp16 scale bits covering normals of both signs, zero, -0 and subnormals."""
    s = np.float16(rng.normal(0, 0.01, n)).view(np.uint16).copy()
    s[::17] = 0x0000
    s[1::17] = 0x8000
    s[2::17] = rng.integers(1, 0x3FF, s[2::17].size)            # subnormal
    s[3::17] = 0x8000 | rng.integers(1, 0x3FF, s[3::17].size)   # negative subnormal
    s[4::17] = 0xBC00                                           # -1.0
    return s


@pytest.mark.parametrize("nblocks", [1, 7, 4096])
def test_q4_0_dequant_bit_exact(rocm, dev, oracle, nblocks):
    rng = np.random.default_rng(nblocks)
    blocks = rng.integers(0, 256, (nblocks, 18), dtype=np.uint8)
    blocks[:, :2] = _random_f16_scales(rng, nblocks).view(np.uint8).reshape(-1, 2)
    blocks[0, 2:] = 0x88                                        # zero codes
    src = dev.put(blocks.ravel())
    out = dev.empty(nblocks * 32)
    rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(src), None, nblocks * 32, rocm.TYPE_Q4_0, 0)
    exp = oracle.dequant(oracle.QTYPE_Q4_0, blocks.ravel(), nblocks * 32)
    assert np.array_equal(_bits(dev.get(out)), _bits(exp))


@pytest.mark.parametrize("nblocks", [1, 5, 4096])
def test_q8_0_dequant_bit_exact(rocm, dev, oracle, nblocks):
    rng = np.random.default_rng(100 + nblocks)
    blocks = rng.integers(0, 256, (nblocks, 34), dtype=np.uint8)
    blocks[:, :2] = _random_f16_scales(rng, nblocks).view(np.uint8).reshape(-1, 2)
    src = dev.put(blocks.ravel())
    out = dev.empty(nblocks * 32)
    rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(src), None, nblocks * 32, rocm.TYPE_Q8_0, 0)
    exp = oracle.dequant(oracle.QTYPE_Q8_0, blocks.ravel(), nblocks * 32)
    assert np.array_equal(_bits(dev.get(out)), _bits(exp))


@pytest.mark.parametrize("numel,group", [(4096 * 64, 64), (1000, 64), (999, 64), (4096, 128), (96, 6)])
def test_nf4_dequant_bit_exact(rocm, dev, oracle, numel, group):
    rng = np.random.default_rng(numel + group)
    codes = rng.integers(0, 256, (numel + 1) // 2, dtype=np.uint8)
    absmax = rng.uniform(0.0, 0.1, (numel + group - 1) // group).astype(np.float32)
    absmax[::11] = 0.0
    absmax[1::11] = np.float32(1e-40)                       # fp32 subnormal scale
    c, a = dev.put(codes), dev.put(absmax)
    out = dev.empty(numel)
    rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(c), dev.ptr(a), numel, rocm.TYPE_NF4, group)
    exp = oracle.nf4_dequant(codes, absmax, numel, group)
    assert np.array_equal(_bits(dev.get(out)), _bits(exp))


def test_f16_dequant_exhaustive(rocm, dev, oracle):
    bits = np.arange(65536, dtype=np.uint16)
    src = dev.put(bits)
    out = dev.empty(65536)
    rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(src), None, 65536, rocm.TYPE_F16, 0)
    exp = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    assert np.array_equal(_bits(dev.get(out)), _bits(exp))


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_gguf_encoders_bit_exact(rocm, dev, oracle, qtype):
    n = 32 * 8192
    w = oracle.normal(7, n, 0.0, 0.02)
    w[:32] = 0.0                                             # all-zero block -> scale 0
    w[32:64] = np.linspace(-7, 7, 32, dtype=np.float32)      # exact ties for Math.round
    t = {"q4_0": (rocm.TYPE_Q4_0, oracle.QTYPE_Q4_0, 18), "q8_0": (rocm.TYPE_Q8_0, oracle.QTYPE_Q8_0, 34)}[qtype]
    src = dev.put(w)
    out = dev.empty(n // 32 * t[2], np.uint8)
    rocm.call("aljabr_rocm_quantize", dev.ptr(out), None, dev.ptr(src), n, t[0], 0)
    assert np.array_equal(dev.get(out), oracle.quantize(t[1], w))


@pytest.mark.parametrize("numel,group", [(64 * 4096, 64), (1000, 64), (999, 64)])
def test_nf4_encoder_bit_exact(rocm, dev, oracle, numel, group):
    w = oracle.normal(numel, numel, 0.0, 0.02)
    w[:group] = 0.0
    src = dev.put(w)
    codes = dev.empty((numel + 1) // 2, np.uint8)
    absmax = dev.empty((numel + group - 1) // group)
    rocm.call("aljabr_rocm_quantize", dev.ptr(codes), dev.ptr(absmax), dev.ptr(src), numel, rocm.TYPE_NF4, group)
    ec, ea = oracle.nf4_quantize(w, group)
    assert np.array_equal(dev.get(codes), ec)
    assert np.array_equal(_bits(dev.get(absmax)), _bits(ea))


def test_f16_encoder_matches_writer(rocm, dev, oracle):
    w = np.concatenate([oracle.normal(3, 4096), np.array([1 + 2 ** -11, 70000.0, 2 ** -24, 2 ** -26], np.float32)])
    src = dev.put(w)
    out = dev.empty(w.size, np.uint16)
    rocm.call("aljabr_rocm_quantize", dev.ptr(out), None, dev.ptr(src), w.size, rocm.TYPE_F16, 0)
    exp = np.array([oracle.f32_to_f16_writer(float(v)) for v in w], dtype=np.uint16)
    assert np.array_equal(dev.get(out).view(np.uint16), exp)


def test_bad_arguments_are_rejected(rocm, dev):
    out = dev.empty(64)
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(out), None, 33, rocm.TYPE_Q4_0, 0)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_dequantize", dev.ptr(out), dev.ptr(out), None, 32, 77, 0)
    assert e.value.status == rocm.ERR_UNSUPPORTED
