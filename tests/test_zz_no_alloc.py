"""aljabr_rocm_attention_gqa_noalloc (the allocation-free variant of
aljabr_rocm_attention_gqa, partials in a static device array) against the
allocating entry point on the same inputs: two calls in a row, the second
smaller than the first, each within the attention tolerance of the
allocating call (1e-3 relative L2; equal split counts give equal bits), plus
the size and mask refusals."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _case(dev, oracle, b, hq, hkv, s, d, seed):
    q = oracle.normal(seed, b * hq * d).reshape(b, hq, 1, d)
    k = oracle.normal(seed + 1, b * hkv * s * d).astype(np.float16)
    v = oracle.normal(seed + 2, b * hkv * s * d).astype(np.float16)
    return [dev.put(q), dev.put(k.view(np.int16)), dev.put(v.view(np.int16))]


def _run(rocm, dev, fn, bufs, b, hq, hkv, s, d):
    out = dev.put(np.full(b * hq * d, np.nan, np.float32))
    rocm.call(fn, dev.ptr(out), *[dev.ptr(t) for t in bufs], None, b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
    return dev.get(out)


def test_noalloc_matches_allocating_entry_point(rocm, dev, oracle):
    # First call: B=2, S=3000 (many splits); second: B=1, S=700, smaller, so
    # its partial slots are a prefix of what the first call left behind.
    for (b, hq, hkv, s, d, seed) in [(2, 32, 8, 3000, 128, 11), (1, 32, 8, 700, 128, 21)]:
        bufs = _case(dev, oracle, b, hq, hkv, s, d, seed)
        ref = _run(rocm, dev, "aljabr_rocm_attention_gqa", bufs, b, hq, hkv, s, d)
        got = _run(rocm, dev, "aljabr_rocm_attention_gqa_noalloc", bufs, b, hq, hkv, s, d)
        assert np.all(np.isfinite(got))
        assert rel_l2(got, ref) <= 1e-5, (b, s)


def test_noalloc_refuses_what_it_cannot_hold(rocm, dev):
    y = dev.empty(64)
    with pytest.raises(rocm.RocmError) as e:      # 64*32*64 rows x 2 x 130 floats > 8 MiB
        rocm.call("aljabr_rocm_attention_gqa_noalloc", dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y), None,
                  64, 32, 8, 64, 64, 128, rocm.TYPE_F16, 0.0, 1)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_attention_gqa_noalloc", dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y),
                  1, 1, 1, 1, 4, 64, rocm.TYPE_F32, 0.0, 0)
    assert e.value.status == rocm.ERR_UNSUPPORTED
