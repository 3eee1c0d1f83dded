"""Concurrent callers of the C ABI: several host threads, each with distinct
inputs, call the library at once (each thread gets its own stream and its
own scratch), and every output equals the oracle's. The reference holds its
Metal bridge to the same contract (MetalTripleBatchCorrectnessTest.java:171-268:
4 workers x 3 iterations of the triple-batch matvec); here each worker also
runs an NF4 matvec and a split-K GQA attention, whose partial results live
in per-stream scratch."""
from __future__ import annotations

import threading

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14
WORKERS, ITERS = 4, 3


def test_concurrent_callers_get_independent_results(rocm, dev, oracle):
    k, ns, batch = 2048, (1024, 256, 256), 3
    nk, nn = 4096, 2048
    b, hq, hkv, s, d = 2, 32, 8, 700, 128
    cases = []
    for w in range(WORKERS):
        seed = 1000 * (w + 1)
        mats = [oracle.random_k_blocks(t, n * k // 256, seed + i, scale=0.5 / np.sqrt(k) / (200 if t == Q4_K else 1000))
                for i, (t, n) in enumerate(zip((Q4_K, Q4_K, Q6_K), ns))]
        x = oracle.normal(seed + 5, batch * k)
        tri_ref = [oracle.q_matvec(t, m, x, n, k).reshape(batch, n) for t, m, n in zip((Q4_K, Q4_K, Q6_K), mats, ns)]
        codes, absmax = oracle.nf4_quantize(oracle.normal(seed + 6, nn * nk, 0.0, 0.02), 64)
        xn = oracle.normal(seed + 7, nk)
        nf4_ref = oracle.nf4_matvec(codes, absmax, xn, nn, nk, 64)
        q = oracle.normal(seed + 8, b * hq * d).reshape(b, hq, 1, d)
        kk = oracle.normal(seed + 9, b * hkv * s * d).astype(np.float16)
        vv = oracle.normal(seed + 10, b * hkv * s * d).astype(np.float16)
        att_ref = oracle.attention_gqa(q, kk.astype(np.float32).reshape(b, hkv, s, d),
                                       vv.astype(np.float32).reshape(b, hkv, s, d), None, True)
        cases.append(dict(
            mats=[dev.put(m) for m in mats], x=dev.put(x), ys=[dev.empty(batch * n) for n in ns], tri_ref=tri_ref,
            codes=dev.put(codes), absmax=dev.put(absmax), xn=dev.put(xn), yn=dev.empty(nn), nf4_ref=nf4_ref,
            q=dev.put(q), k=dev.put(kk.view(np.int16)), v=dev.put(vv.view(np.int16)), out=dev.empty(b * hq * d),
            att_ref=att_ref, results=[], error=None))

    start = threading.Barrier(WORKERS)

    def worker(c):
        try:
            start.wait()
            for _ in range(ITERS):
                rocm.call("aljabr_rocm_matvec_tb_triple_batch", *[dev.ptr(y) for y in c["ys"]], dev.ptr(c["x"]),
                          *[dev.ptr(m) for m in c["mats"]], k, *ns, Q4_K, Q4_K, Q6_K, batch)
                rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(c["yn"]), dev.ptr(c["xn"]), dev.ptr(c["codes"]),
                          dev.ptr(c["absmax"]), nk, nn, 64)
                rocm.call("aljabr_rocm_attention_gqa", dev.ptr(c["out"]), dev.ptr(c["q"]), dev.ptr(c["k"]),
                          dev.ptr(c["v"]), None, b, hq, hkv, 1, s, d, rocm.TYPE_F16, 0.0, 1)
                # The calls are synchronous on the thread's stream: the
                # outputs are complete when they return.
                c["results"].append(([y.cpu().numpy() for y in c["ys"]], c["yn"].cpu().numpy(),
                                     c["out"].cpu().numpy()))
        except Exception as e:          # reported by the main thread
            c["error"] = e

    threads = [threading.Thread(target=worker, args=(c,)) for c in cases]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    for w, c in enumerate(cases):
        assert c["error"] is None, (w, c["error"])
        assert len(c["results"]) == ITERS, w
        for it, (tri, yn, out) in enumerate(c["results"]):
            for got, want, n in zip(tri, c["tri_ref"], ns):
                got = got.reshape(batch, n)
                for r in range(batch):
                    assert rel_l2(got[r], want[r]) <= 1e-3, (w, it, r)
            assert rel_l2(yn, c["nf4_ref"]) <= 1e-3, (w, it)
            assert rel_l2(out, c["att_ref"]) <= 1e-3, (w, it)
