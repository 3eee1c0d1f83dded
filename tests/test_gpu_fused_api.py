"""GPU parity of the multi-matrix entry points (the Metal ABI's matvec pair,
triple, triple batch and gated FFN; MTLC/aljabr_metal_matvec_api.h:83-120)
against the oracle on identical seeded inputs: each output within 1e-3
relative L2. One-type sets take one stacked launch (rows kernel at batch 1,
matrix cores at batch >= 2); mixed types one launch per matrix."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14


def _matrix(oracle, t, n, k, seed):
    """(raw weights for the device, oracle matvec callable)."""
    if t in (Q4_K, Q6_K):
        raw = oracle.random_k_blocks(t, n * k // 256, seed, scale=0.5 / np.sqrt(k) / (200 if t == Q4_K else 1000))
        return raw, lambda x, m: oracle.q_matvec(t, raw, x, n, k).reshape(m, n)
    w = oracle.normal(seed, n * k, 0.0, 0.5 / np.sqrt(k))
    if t in (Q4_0, Q8_0):
        raw = oracle.quantize(t, w)
        return raw, lambda x, m: oracle.q_matvec(t, raw, x, n, k).reshape(m, n)
    if t == F16:
        raw = w.astype(np.float16).view(np.uint16)
        return raw, lambda x, m: oracle.f16_matvec(raw, x, n, k).reshape(m, n)
    raw = w.astype(np.float32)
    return raw, lambda x, m: (x.reshape(m, k).astype(np.float64) @ raw.reshape(n, k).T.astype(np.float64)).astype(
        np.float32)


@pytest.mark.parametrize("types,k,ns", [((Q4_0, Q4_0), 4096, (1536, 1536)), ((Q4_K, Q4_K), 4096, (1024, 512)),
                                        ((Q8_0, Q6_K), 2048, (640, 384)), ((F16, F32), 512, (300, 200))])
def test_pair(rocm, dev, oracle, types, k, ns):
    mats = [_matrix(oracle, t, n, k, 11 + i) for i, (t, n) in enumerate(zip(types, ns))]
    x = oracle.normal(5, k)
    ys = [dev.empty(n) for n in ns]
    ws = [dev.put(m[0]) for m in mats]
    xd = dev.put(x)                     # kept alive until the call has run
    rocm.call("aljabr_rocm_matvec_tb_pair", dev.ptr(ys[0]), dev.ptr(ys[1]), dev.ptr(xd), dev.ptr(ws[0]),
              dev.ptr(ws[1]), k, ns[0], ns[1], types[0], types[1])
    for y, (_, ref) in zip(ys, mats):
        assert rel_l2(dev.get(y), ref(x, 1).ravel()) <= 1e-3


@pytest.mark.parametrize("types,batch", [((Q4_K, Q4_K, Q4_K), 1), ((Q8_0, Q8_0, Q8_0), 1), ((Q4_K, Q4_K, Q4_K), 4),
                                         ((Q4_0, Q4_0, Q4_0), 6), ((Q6_K, Q4_K, Q6_K), 3), ((F16, F16, F16), 2)])
def test_triple(rocm, dev, oracle, types, batch):
    k, ns = 2048, (1024, 256, 256)
    mats = [_matrix(oracle, t, n, k, 31 + i) for i, (t, n) in enumerate(zip(types, ns))]
    x = oracle.normal(7 + batch, batch * k)
    ys = [dev.empty(batch * n) for n in ns]
    ws = [dev.put(m[0]) for m in mats]
    xd = dev.put(x)
    if batch == 1:
        rocm.call("aljabr_rocm_matvec_tb_triple", *[dev.ptr(y) for y in ys], dev.ptr(xd), *[dev.ptr(w) for w in ws],
                  k, *ns, *types)
    else:
        rocm.call("aljabr_rocm_matvec_tb_triple_batch", *[dev.ptr(y) for y in ys], dev.ptr(xd),
                  *[dev.ptr(w) for w in ws], k, *ns, *types, batch)
    for y, n, (_, ref) in zip(ys, ns, mats):
        got = dev.get(y).reshape(batch, n)
        want = ref(x, batch)
        for b in range(batch):
            assert rel_l2(got[b], want[b]) <= 1e-3, b


@pytest.mark.parametrize("types,kind,batch", [((Q4_K, Q4_K, Q6_K), 1, 1), ((Q4_0, Q4_0, Q8_0), 0, 1),
                                              ((Q4_K, Q4_K, Q6_K), 2, 3), ((F16, Q8_0, F32), 1, 2)])
def test_ffn_gated_fused(rocm, dev, oracle, types, kind, batch):
    dim, ffn = 1024, 2048
    g, u, d = (_matrix(oracle, t, n, k, 51 + i) for i, (t, n, k) in enumerate(zip(types, (ffn, ffn, dim),
                                                                                    (dim, dim, ffn))))
    x = oracle.normal(9, batch * dim)
    out = dev.empty(batch * dim)
    bufs = [dev.put(a) for a in (x, g[0], u[0], d[0])]   # kept alive until the call has run
    args = [dev.ptr(out), *[dev.ptr(t) for t in bufs], dim, ffn, *types, kind]
    if batch == 1:
        rocm.call("aljabr_rocm_ffn_gated_fused", *args)
    else:
        rocm.call("aljabr_rocm_ffn_gated_fused_batch", *args, batch)
    h = oracle.gated_activation(g[1](x, batch), u[1](x, batch), kind)
    want = d[1](np.ascontiguousarray(h.ravel()), batch)
    got = dev.get(out).reshape(batch, dim)
    for b in range(batch):
        assert rel_l2(got[b], want[b]) <= 1e-3, b


def test_argument_errors(rocm, dev):
    from aljabr_amd import abi
    x = dev.empty(64)
    with pytest.raises(abi.RocmError) as e:
        rocm.call("aljabr_rocm_matvec_tb_pair", dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), 48, 1, 1,
                  Q4_0, Q4_0)
    assert e.value.status == abi.ERR_BAD_ARGUMENT
    with pytest.raises(abi.RocmError) as e:
        rocm.call("aljabr_rocm_matvec_tb_pair", dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), dev.ptr(x), 64, 1, 1,
                  Q4_0, 13)
    assert e.value.status == abi.ERR_UNSUPPORTED
