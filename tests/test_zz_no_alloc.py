"""aljabr_rocm_attention_gqa_noalloc (the allocation-free variant of
aljabr_rocm_attention_gqa, partials in a static device array) against the
allocating entry point on the same inputs: two calls in a row, the second
smaller than the first, each within 1e-5 relative L2 of the allocating call
(equal split counts give equal bits). The no-alloc calls run first, on a
fresh thread (a stream no call has used yet): the device's free memory and
the stream's library scratch stay as they were. (The thread first runs one
plain element-wise kernel: the thread's first call creates its stream, and
the runtime sets up a stream's queue at its first launch.) Plus the size
and mask refusals."""
from __future__ import annotations

import ctypes
import threading

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
    import torch
    # First call: B=2, S=3000 (many splits); second: B=1, S=700, smaller, so
    # its partial slots are a prefix of what the first call left behind.
    cases = [(2, 32, 8, 3000, 128, 11), (1, 32, 8, 700, 128, 21)]
    bufs = [_case(dev, oracle, *c) for c in cases]
    outs = [dev.put(np.full(c[0] * c[1] * c[4], np.nan, np.float32)) for c in cases]
    seen = {}

    def noalloc_calls():
        try:
            held = ctypes.c_size_t(1)
            warm = dev.empty(64)
            rocm.call("aljabr_rocm_add_inplace", dev.ptr(warm), dev.ptr(warm), 64)
            free0 = torch.cuda.mem_get_info(0)[0]
            for (b, hq, hkv, s, d, _), bf, out in zip(cases, bufs, outs):
                rocm.call("aljabr_rocm_attention_gqa_noalloc", dev.ptr(out), *[dev.ptr(t) for t in bf], None,
                          b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
            rocm.call("aljabr_rocm_stream_scratch_bytes", ctypes.byref(held))
            seen.update(free=torch.cuda.mem_get_info(0)[0] - free0, held=held.value)
        except BaseException as e:               # reported on the test's thread
            seen.update(error=repr(e))

    t = threading.Thread(target=noalloc_calls)
    t.start()
    t.join(timeout=120)
    assert not t.is_alive(), "the no-alloc thread did not finish"
    assert seen == {"free": 0, "held": 0}
    for (b, hq, hkv, s, d, _), bf, out in zip(cases, bufs, outs):
        got = dev.get(out)
        ref = _run(rocm, dev, "aljabr_rocm_attention_gqa", bf, b, hq, hkv, s, d)
        assert np.all(np.isfinite(got))
        assert rel_l2(got, ref) <= 1e-5, (b, s)


def test_noalloc_refuses_what_it_cannot_hold(rocm, dev):
    y = dev.empty(64)
    with pytest.raises(rocm.RocmError) as e:      # 64*32*64 rows x 2 x 130 floats > an 8 MiB slot
        rocm.call("aljabr_rocm_attention_gqa_noalloc", dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y), None,
                  64, 32, 8, 64, 64, 128, rocm.TYPE_F16, 0.0, 1)
    assert e.value.status == rocm.ERR_BAD_ARGUMENT
    with pytest.raises(rocm.RocmError) as e:
        rocm.call("aljabr_rocm_attention_gqa_noalloc", dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y), dev.ptr(y),
                  1, 1, 1, 1, 4, 64, rocm.TYPE_F32, 0.0, 0)
    assert e.value.status == rocm.ERR_UNSUPPORTED
