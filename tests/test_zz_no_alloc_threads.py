"""aljabr_rocm_attention_gqa_noalloc from two threads at once: each thread has
its own library stream and so its own slot of the static partials array, and
every call of both threads equals the allocating entry point's output for the
same inputs (computed beforehand on the main thread) bit for bit (the slot
holds every split the allocating call would use). Without per-stream slots
the two streams' split kernels would overwrite each other's partials."""
from __future__ import annotations

import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (B, Hq, Hkv, S, D): different shapes per thread, so partials that leaked
# from the other thread's call could not go unnoticed.
SHAPES = [(2, 32, 8, 3000, 128), (1, 32, 8, 1800, 128)]
ROUNDS = 40


def _inputs(dev, oracle, b, hq, hkv, s, d, seed):
    q = oracle.normal(seed, b * hq * d)
    k = oracle.normal(seed + 1, b * hkv * s * d).astype(np.float16)
    v = oracle.normal(seed + 2, b * hkv * s * d).astype(np.float16)
    return [dev.put(q), dev.put(k.view(np.int16)), dev.put(v.view(np.int16))]


def test_two_threads_do_not_share_partials(rocm, dev, oracle):
    import torch
    cases = []
    for i, (b, hq, hkv, s, d) in enumerate(SHAPES):
        bufs = _inputs(dev, oracle, b, hq, hkv, s, d, 100 + 10 * i)
        out = dev.empty(b * hq * d)
        rocm.call("aljabr_rocm_attention_gqa", dev.ptr(out), *[dev.ptr(t) for t in bufs], None,
                  b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
        cases.append((bufs, (b, hq, hkv, s, d), dev.get(out)))

    errors, start = [], threading.Barrier(len(cases))

    def worker(idx):
        try:
            bufs, (b, hq, hkv, s, d), ref = cases[idx]
            outs = [torch.full((b * hq * d,), float("nan"), dtype=torch.float32, device="cuda:0")
                    for _ in range(ROUNDS)]
            torch.cuda.synchronize()
            # Stream-ordered calls: the thread's work queues up and overlaps
            # the other thread's on the GPU.
            rocm.call("aljabr_rocm_set_sync_mode", 0)
            start.wait()
            for r in range(ROUNDS):
                rocm.call("aljabr_rocm_attention_gqa_noalloc", outs[r].data_ptr(), *[t.data_ptr() for t in bufs],
                          None, b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
            rocm.call("aljabr_rocm_synchronize")
            rocm.call("aljabr_rocm_set_sync_mode", 1)
            for r in range(ROUNDS):
                got = outs[r].cpu().numpy()
                if not np.array_equal(got, ref):
                    errors.append(f"thread {idx} call {r}: max |diff| {np.nanmax(np.abs(got - ref))}")
                    return
        except BaseException as e:               # reported on the test's thread
            errors.append(f"thread {idx}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
