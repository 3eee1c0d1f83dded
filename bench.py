"""Headline benchmark: NF4 dequant-fused matvec HBM GB/s at Llama-3-8B MLP
shapes on one MI355X, plus the Llama-3-8B-shaped NF4 decode tokens/s.

A step is one pass of the hot path over one batch: the three MLP projections of
one Llama-3-8B layer at batch 1 (gate 14336x4096, up 14336x4096, down
4096x14336; NF4, block 64, fp32 absmax, fp32 activations)
configs[1] at M=1. Weights rotate through enough distinct copies (>= 512 MB)
that the Infinity Cache cannot serve them; all inputs are resident in HBM
before the timed region. `value` is algorithmic bytes moved per second.

Prints ONE JSON line. `python bench.py --gpus N --steps K --warmup W`.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TF = 2500.0   # MI355X dense fp16 matrix-core peak
K_MODEL, FFN = 4096, 14336
BLOCK = 64
KERNEL = "rows_kernel"              # the batch-1 kernel these launches dispatch to (matvec_rows.hip)


def nf4_bytes(n: int, k: int, m: int = 1) -> int:
    """Algorithmic bytes of one NF4 matvec: codes + absmax + x + y."""
    return n * k // 2 + (n * k // BLOCK) * 4 + m * k * 4 + m * n * 4


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# A timed region's launches go out from Python through ctypes at ~4.5 us each
# (more right after a synchronize), the order of one of the kernels timed
# here (4-9 us). Started on an idle GPU, a region therefore also times the
# host's enqueue rate: the GPU waits for the first launch and then runs on a
# queue only a launch or two deep. A GPU spin queued on the stream just
# before the start event (~0.4 ms at 2.4 GHz) lets the host enqueue the
# region's launches while the GPU is busy; the start event fires when the
# spin ends, so the region times exactly its launches, back to back.
HEAD_START_CYCLES = 1_000_000


def head_start(torch) -> None:
    """Queue the untimed GPU spin on the current stream (call right before a
    timed region's start event, after any synchronize)."""
    torch.cuda._sleep(HEAD_START_CYCLES)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed MLP steps right before the timed ones")
    ap.add_argument("--clock-warmup-ms", type=float, default=300.0,
                    help="untimed MLP steps for at least this long before the --warmup steps (the GPU needs "
                         "~15 ms of load to reach its steady clocks); reported as clock_warmup_ms")
    ap.add_argument("--section-pause-s", type=float, default=2.0,
                    help="idle seconds before each later section of the default run, so that none is timed in the "
                         "slowed state a long memory-bound section leaves behind (each section then runs its own "
                         "untimed warm-up launches); reported as section_pause_s")
    ap.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0: enough for 512 MB)")
    ap.add_argument("--no-decode", action="store_true", help="skip the Llama decode measurement")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--decode-steps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the small-M GEMM and attention measurements (BASELINE configs 2 and 4)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 256 MiB device copy 20 times (FETCH_SIZE/WRITE_SIZE calibration)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode-step measurement (for profiling runs; prints its own JSON line)")
    ap.add_argument("--gguf-decode-only", action="store_true",
                    help="run only the GGUF Q4_K_M decode measurement (for profiling)")
    ap.add_argument("--kquant-only", action="store_true",
                    help="run only the GGUF Q4_0/Q8_0 and K-quant matvec/GEMM measurements (for profiling)")
    ap.add_argument("--small-m-only", action="store_true",
                    help="run only the NF4 small-M GEMM measurement (for profiling)")
    ap.add_argument("--small-m", type=str, default="1,4,16,32,64",
                    help="with --small-m-only: the token counts M to time (comma-separated)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the prefill attention measurement (for profiling)")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the GQA decode attention measurement (for profiling)")
    ap.add_argument("--step-only", action="store_true",
                    help="run only the registered whole-step (Metal ABI) decode measurement")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="only time a plain streaming read of rotating 33 MB buffers (the batch-1 ceiling)")
    ap.add_argument("--ceiling-workgroups", type=int, default=0,
                    help="with --stream-ceiling: only this workgroup count (0: the sweep)")
    return ap.parse_args()


def make_mlp_copies(abi, torch, copies: int):
    from aljabr_amd.llama import nf4_quantize_device
    g = torch.Generator(device="cuda:0").manual_seed(2024)
    mats = []
    for _ in range(copies):
        layer = []
        for n, k in ((FFN, K_MODEL), (FFN, K_MODEL), (K_MODEL, FFN)):
            w = torch.randn(n * k, generator=g, device="cuda:0").mul_(0.02)
            c, a = nf4_quantize_device(w, BLOCK)
            del w
            layer.append((c, a, n, k))
        mats.append(layer)
    torch.cuda.synchronize()
    return mats


def time_mlp(abi, torch, stream, mats, steps: int, warmup: int, clock_warmup_ms: float, idle_start: bool = False):
    """Milliseconds of `steps` MLP steps, after untimed steps for at least
    `clock_warmup_ms` of wall time and then `warmup` more; returns (ms,
    clock warm-up ms, clock warm-up steps, ms of a second `steps`-step region
    started on an idle GPU without the head start, or None)."""
    lib = abi.load()
    x = torch.randn(K_MODEL, device="cuda:0")
    h = torch.randn(FFN, device="cuda:0")
    outs = [torch.empty(FFN, device="cuda:0"), torch.empty(FFN, device="cuda:0"), torch.empty(K_MODEL, device="cuda:0")]
    ins = [x, x, h]
    torch.cuda.synchronize()

    def step(i):
        for j, (c, a, n, k) in enumerate(mats[i % len(mats)]):
            rc = lib.aljabr_rocm_matvec_tb_nf4(outs[j].data_ptr(), ins[j].data_ptr(), c.data_ptr(), a.data_ptr(),
                                                k, n, BLOCK)
            if rc:
                abi.check(rc, "aljabr_rocm_matvec_tb_nf4")

    with torch.cuda.stream(stream):
        # Clock warm-up: batches of 100 steps until the wall clock says so.
        done, t0 = 0, time.perf_counter()
        while True:
            for _ in range(100):
                step(done)
                done += 1
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= clock_warmup_ms:
                break
        clock_ms = (time.perf_counter() - t0) * 1e3
        for i in range(warmup):
            step(done + i)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        head_start(torch)
        start.record(stream)
        for i in range(steps):
            step(done + warmup + i)
        end.record(stream)
        end.synchronize()
        idle_ms = None
        if idle_start:
            # The same region as it times without the head start.
            torch.cuda.synchronize()
            s2, e2 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s2.record(stream)
            for i in range(steps):
                step(done + warmup + steps + i)
            e2.record(stream)
            e2.synchronize()
            idle_ms = s2.elapsed_time(e2)
    torch.cuda.synchronize()
    return start.elapsed_time(end), clock_ms, done, idle_ms


def _cpu_rate(fn, nbytes: int, seconds: float):
    """Repeat fn() for about `seconds`; returns (GB/s of algorithmic bytes, runs, seconds)."""
    fn()                                          # warm
    done, t0 = 0, time.perf_counter()
    while True:
        fn()
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return nbytes * done / dt / 1e9, done, dt


def cpu_baseline(seconds: float, llama_host=None):
    """The oracle (C restatement of the reference CPU path, OpenMP row chunks =
    2 x threads as GgufParallelConfig) on bounded samples: the NF4 MLP step
    at all host cores for ~`seconds` (the reported value), then single-thread
    and all-core rates of the NF4, Q4_0, Q8_0 and Q4_K matvecs (14336x4096)
    and GQA decode attention (B=1 and 16, S=4096, fp16 K/V widened to fp32)
    for ~2 s each, and, given the Llama-3-8B NF4 model's host weights, two
    batch-1 decode tokens of the whole step at all cores. The reference's own
    Java Vector-API path cannot run here."""
    import numpy as np
    import oracle
    threads = oracle.threads()
    mats = []
    for i, (n, k) in enumerate(((FFN, K_MODEL), (FFN, K_MODEL), (K_MODEL, FFN))):
        codes, absmax = oracle.nf4_quantize(oracle.normal(100 + i, n * k, 0.0, 0.02), BLOCK)
        mats.append((codes, absmax, n, k))
    xs = {K_MODEL: oracle.normal(7, K_MODEL), FFN: oracle.normal(8, FFN)}
    step_bytes = sum(nf4_bytes(n, k) for _, _, n, k in mats)

    def mlp():
        for codes, absmax, n, k in mats:
            oracle.nf4_matvec(codes, absmax, xs[k], n, k, BLOCK, threads)
    gbs, done, dt = _cpu_rate(mlp, step_bytes, seconds)
    extra = {}
    c0, a0 = mats[0][0], mats[0][1]
    for t in (1, threads):
        r, _, _ = _cpu_rate(lambda: oracle.nf4_matvec(c0, a0, xs[K_MODEL], FFN, K_MODEL, BLOCK, t),
                            nf4_bytes(FFN, K_MODEL), 2.0)
        extra[f"nf4_14336x4096_m1_{t}t_GBs"] = round(r, 3)
    w32 = oracle.normal(200, FFN * K_MODEL, 0.0, 0.02)
    for name, qt, q in (("q4_0", oracle.QTYPE_Q4_0, oracle.quantize(oracle.QTYPE_Q4_0, w32)),
                        ("q8_0", oracle.QTYPE_Q8_0, oracle.quantize(oracle.QTYPE_Q8_0, w32)),
                        ("q4_k", oracle.QTYPE_Q4_K, oracle.random_k_blocks(oracle.QTYPE_Q4_K, FFN * K_MODEL // 256,
                                                                           201))):
        for t in (1, threads):
            r, _, _ = _cpu_rate(lambda: oracle.q_matvec(qt, q, xs[K_MODEL], FFN, K_MODEL, t),
                                q.size + 4 * (FFN + K_MODEL), 2.0)
            extra[f"{name}_14336x4096_m1_{t}t_GBs"] = round(r, 3)
    del w32
    hq, hkv, d, s = 32, 8, 128, 4096
    for b in (1, 16):
        qv = oracle.normal(300 + b, b * hq * d).reshape(b, hq, 1, d)
        kv = oracle.normal(310 + b, b * hkv * s * d).astype(np.float16).astype(np.float32).reshape(b, hkv, s, d)
        vv = oracle.normal(320 + b, b * hkv * s * d).astype(np.float16).astype(np.float32).reshape(b, hkv, s, d)
        nbytes = 2 * b * hkv * s * d * 2 + 2 * b * hq * d * 4      # fp16 K/V as the GPU reads them
        for t in (1, threads):
            r, _, _ = _cpu_rate(lambda: oracle.attention_gqa(qv, kv, vv, None, True, t), nbytes, 2.0)
            extra[f"attention_b{b}_s{s}_{t}t_GBs"] = round(r, 3)
    decode = None
    if llama_host is not None:
        from aljabr_amd.llama import LLAMA3_8B
        ref = oracle.LlamaOracle(dict(LLAMA3_8B, max_seq=8), llama_host)
        t0 = time.perf_counter()
        tok, _, _ = ref.decode(17, 0, threads)
        ref.decode(tok, 1, threads)
        dt2 = time.perf_counter() - t0
        decode = {"tokens_per_s": round(2.0 / dt2, 3), "ms_per_token": round(dt2 * 500.0, 1), "cores": threads,
                  "sample": "2 batch-1 decode tokens (positions 0, 1) of the Llama-3-8B NF4 model the GPU decode "
                            "bench runs (32 layers, fp16 LM head), oracle.LlamaOracle at all threads"}
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{done} MLP steps (3 NF4 matvecs each: 14336x4096, 14336x4096, 4096x14336, batch 1), "
                      f"{dt:.1f} s, oracle C restatement, OpenMP row chunks = 2 x {threads} threads",
            "per_kernel": extra,
            "per_kernel_sample": "about 2 s per entry: 1 thread and all host threads; attention bytes count "
                                 "K/V at fp16 (the GPU's format) though the oracle reads them widened",
            "decode_llama3_8b_nf4_b1": decode}


def small_m_bench(abi, torch, stream, ms=(1, 4, 16, 32, 64), launches=60):
    """NF4 small-M GEMM at the MLP shapes, M tokens per
    launch (M <= 4 on the rows kernel in fp32, M >= 5 on the matrix cores),
    and configs[0]'s 4096x4096 matvec at M = 1. Weights rotate over >= 512 MB.
    Returns per-shape, per-M launch time, algorithmic GB/s, TFLOP/s and the
    fraction of HBM peak."""
    lib = abi.load()
    out = {}
    for n, k, mlist in ((K_MODEL, K_MODEL, (1,)), (FFN, K_MODEL, ms), (K_MODEL, FFN, ms)):
        per = n * k // 2 + n * k // BLOCK * 4
        copies = max(2, -(-520_000_000 // per))
        from aljabr_amd.llama import nf4_quantize_device
        g = torch.Generator(device="cuda:0").manual_seed(3)
        bufs = [nf4_quantize_device(torch.randn(n * k, generator=g, device="cuda:0").mul_(0.02), BLOCK)
                for _ in range(copies)]
        for m in mlist:
            x = torch.randn(m * k, device="cuda:0")
            y = torch.empty(m * n, device="cuda:0")
            torch.cuda.synchronize()

            def launch(i):
                c, a = bufs[i % copies]
                rc = lib.aljabr_rocm_matvec_tb_batch_nf4(y.data_ptr(), x.data_ptr(), c.data_ptr(), a.data_ptr(),
                                                         k, n, BLOCK, m)
                if rc:
                    abi.check(rc, "aljabr_rocm_matvec_tb_batch_nf4")
            for i in range(5):
                launch(i)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            head_start(torch)
            start.record(stream)
            for i in range(launches):
                launch(i)
            end.record(stream)
            end.synchronize()
            us = start.elapsed_time(end) * 1000.0 / launches
            alg = per + m * (k + n) * 4
            out[f"{n}x{k}_m{m}"] = {"us": round(us, 2), "GBs": round(alg / us / 1e3, 1),
                                    "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 3),
                                    "TFLOPs": round(2.0 * m * n * k / us / 1e6, 1)}
        del bufs
        torch.cuda.empty_cache()
    return out


def gguf_q_bench(abi, torch, stream, ms=(1, 8), launches=60):
    """GGUF Q4_0 / Q8_0 matvec at 4096x4096 and
    14336x4096 from N(0, 0.02) weights (quantized on the device by the
    GGUFWriter rules), x ~ N(0,1) at batch 1 and 8; weights rotate over
    >= 512 MB. Launch time and algorithmic GB/s (blocks once + activations)."""
    lib = abi.load()
    out = {}
    for qtype, name, bb in ((abi.TYPE_Q4_0, "q4_0", 18), (abi.TYPE_Q8_0, "q8_0", 34)):
        for n, k in ((K_MODEL, K_MODEL), (FFN, K_MODEL)):
            per = n * k // 32 * bb
            copies = max(2, -(-520_000_000 // per))
            g = torch.Generator(device="cuda:0").manual_seed(9)
            bufs = []
            for _ in range(copies):
                w = torch.randn(n * k, generator=g, device="cuda:0").mul_(0.02)
                q = torch.empty(per, dtype=torch.uint8, device="cuda:0")
                torch.cuda.synchronize()
                abi.call("aljabr_rocm_quantize", q.data_ptr(), None, w.data_ptr(), n * k, qtype, 0)
                abi.call("aljabr_rocm_synchronize")
                del w
                bufs.append(q)
            for m in ms:
                x = torch.randn(m * k, device="cuda:0")
                y = torch.empty(m * n, device="cuda:0")
                torch.cuda.synchronize()

                def launch(i):
                    rc = lib.aljabr_rocm_matvec_tb_batch(y.data_ptr(), x.data_ptr(), bufs[i % copies].data_ptr(),
                                                         k, n, qtype, m)
                    if rc:
                        abi.check(rc, "aljabr_rocm_matvec_tb_batch")
                for i in range(20):
                    launch(i)
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                head_start(torch)
                start.record(stream)
                for i in range(launches):
                    launch(i)
                end.record(stream)
                end.synchronize()
                us = start.elapsed_time(end) * 1000.0 / launches
                alg = per + m * (k + n) * 4
                out[f"{name}_{n}x{k}_m{m}"] = {"us": round(us, 2), "GBs": round(alg / us / 1e3, 1),
                                               "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 3)}
            del bufs
            torch.cuda.empty_cache()
    return out


def kquant_blocks(torch, qtype, n, k, g):
    """Synthetic GGUF Q4_K (type 12) / Q6_K (14) rows on the device: every code
    byte uniform, fp16 block scales finite and ~1/256 (dmin >= 0)."""
    bb = 144 if qtype == 12 else 210
    nb = n * k // 256
    b = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device="cuda:0", generator=g)
    d = (torch.rand(nb, generator=g, device="cuda:0") * 0.75 + 0.25).mul_(1.0 / 256).half()
    if qtype == 12:
        dmin = torch.rand(nb, generator=g, device="cuda:0").mul_(1.0 / 256).half()
        b[:, 0:2] = d.view(torch.uint8).view(nb, 2)
        b[:, 2:4] = dmin.view(torch.uint8).view(nb, 2)
    else:
        b[:, 208:210] = d.view(torch.uint8).view(nb, 2)
    return b.view(-1)


def kquant_bench(abi, torch, stream, ms=(1, 4, 8), launches=60):
    """GGUF K-quant matvec / small-M GEMM (the quantization of production GGUF
    files) at the Llama-3-8B MLP shapes; weights rotate over >= 512 MB.
    Returns per type, shape and M the launch time and algorithmic GB/s
    (weight blocks once + activations in and out)."""
    lib = abi.load()
    out = {}
    for qtype, name, bb in ((12, "q4_k", 144), (14, "q6_k", 210)):
        for n, k in ((FFN, K_MODEL), (K_MODEL, FFN)):
            per = n * k // 256 * bb
            copies = max(2, -(-520_000_000 // per))
            g = torch.Generator(device="cuda:0").manual_seed(5)
            bufs = [kquant_blocks(torch, qtype, n, k, g) for _ in range(copies)]
            for m in ms:
                x = torch.randn(m * k, device="cuda:0")
                y = torch.empty(m * n, device="cuda:0")
                torch.cuda.synchronize()

                def launch(i):
                    rc = lib.aljabr_rocm_matvec_tb_batch(y.data_ptr(), x.data_ptr(), bufs[i % copies].data_ptr(),
                                                         k, n, qtype, m)
                    if rc:
                        abi.check(rc, "aljabr_rocm_matvec_tb_batch")
                for i in range(20):
                    launch(i)
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                head_start(torch)
                start.record(stream)
                for i in range(launches):
                    launch(i)
                end.record(stream)
                end.synchronize()
                us = start.elapsed_time(end) * 1000.0 / launches
                alg = per + m * (k + n) * 4
                out[f"{name}_{n}x{k}_m{m}"] = {"us": round(us, 2), "GBs": round(alg / us / 1e3, 1),
                                               "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 3)}
            del bufs
            torch.cuda.empty_cache()
    return out


def attention_bench(abi, torch, stream, launches=20):
    """GQA decode attention, Hq=32, Hkv=8, D=128, fp16
    K/V ~N(0,1), one query token per sequence, scale 1/sqrt(128). Small
    configurations rotate through a >= 1 GiB K/V pool so the caches cannot
    serve them. Returns launch time and algorithmic GB/s (K + V + Q + O)."""
    lib = abi.load()
    hq, hkv, d = 32, 8, 128
    out = {}
    pool_elems = 1 << 29                                   # 1 GiB of fp16 per K and V pool
    for b, sk in ((1, 512), (16, 512), (64, 512), (1, 4096), (16, 4096), (64, 4096), (1, 32768), (16, 32768),
                  (64, 32768)):
        kv = b * hkv * sk * d
        elems = max(kv, pool_elems)
        kpool = torch.randn(elems, device="cuda:0", dtype=torch.float16)
        vpool = torch.randn(elems, device="cuda:0", dtype=torch.float16)
        q = torch.randn(b * hq * d, device="cuda:0")
        o = torch.empty(b * hq * d, device="cuda:0")
        slots = max(1, elems // kv)
        torch.cuda.synchronize()

        def launch(i):
            off = (i % slots) * kv * 2
            rc = lib.aljabr_rocm_attention_gqa(o.data_ptr(), q.data_ptr(), kpool.data_ptr() + off,
                                               vpool.data_ptr() + off, None, b, hq, hkv, 1, sk, d,
                                               abi.TYPE_F16, 0.0, 1)
            if rc:
                abi.check(rc, "aljabr_rocm_attention_gqa")
        for i in range(3):
            launch(i)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        head_start(torch)
        start.record(stream)
        for i in range(launches):
            launch(i)
        end.record(stream)
        end.synchronize()
        us = start.elapsed_time(end) * 1000.0 / launches
        alg = 2 * kv * 2 + 2 * b * hq * d * 4
        out[f"b{b}_s{sk}"] = {"us": round(us, 2), "GBs": round(alg / us / 1e3, 1)}
        del kpool, vpool
        torch.cuda.empty_cache()
    return out


def prefill_bench(abi, torch, stream, launches=5):
    """Prefill (FA4) attention at the Llama-3-8B head layout: B = 1, 32 query
    heads over 8 KV heads, D = 128, causal, T = S, fp32 Q/K/V ~ N(0,1),
    scale 1/sqrt(128). Algorithmic flops = 4 * D * H * (visible (query, key)
    pairs), against the fp16 dense matrix-core peak (the kernel issues three
    fp16 MFMAs per product for fp32 accuracy)."""
    lib = abi.load()
    h, hkv, d = 32, 8, 128
    out = {}
    for t in (512, 2048, 8192):
        q = torch.randn(t * h * d, device="cuda:0")
        k = torch.randn(t * hkv * d, device="cuda:0")
        v = torch.randn(t * hkv * d, device="cuda:0")
        o = torch.empty_like(q)
        torch.cuda.synchronize()

        def launch():
            rc = lib.aljabr_rocm_fa4_attention(o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, t, t, h,
                                               hkv, d, 1.0 / math.sqrt(d), 1, 0, 0.0)
            if rc:
                abi.check(rc, "aljabr_rocm_fa4_attention")
        launch()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        head_start(torch)
        start.record(stream)
        for _ in range(launches):
            launch()
        end.record(stream)
        end.synchronize()
        us = start.elapsed_time(end) * 1000.0 / launches
        pairs = t * (t + 1) // 2
        flops = 4.0 * d * h * pairs
        tf = flops / us / 1e6
        out[f"t{t}"] = {"us": round(us, 1), "TFLOPs": round(tf, 1), "frac_fp16_peak": round(tf / MFMA_F16_PEAK_TF, 4)}
        del q, k, v, o
        torch.cuda.empty_cache()
    return out


def traffic_record(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor), or
    None when no summary for this kernel is committed."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return int(rec["bytes_per_launch"]) if rec else None


CEILING_BYTES = FFN * K_MODEL // 2 + FFN * K_MODEL // BLOCK * 4   # codes + absmax of one 14336x4096 matrix


def stream_ceiling(abi, torch, stream, launches: int = 300, wgs=(256, 512, 1024, 2048, 4096, 8192)):
    """A plain streaming read (aljabr_rocm_stream_read_probe) of rotating
    buffers of one NF4 14336x4096 matrix's bytes (codes + absmax, 33,030,144
    B), enough of them for 512 MB as the MLP step rotates its copies: the
    read-only rate one launch of that size reaches, per workgroup count."""
    lib = abi.load()
    copies = max(2, -(-512_000_000 // CEILING_BYTES))
    bufs = [torch.randint(0, 255, (CEILING_BYTES,), dtype=torch.uint8, device="cuda:0") for _ in range(copies)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda:0")
    torch.cuda.synchronize()
    out = {"bytes_per_launch": CEILING_BYTES, "copies": copies, "launches": launches, "by_workgroups": {}}
    best = None
    with torch.cuda.stream(stream):
        for wg in wgs:
            def go(i):
                rc = lib.aljabr_rocm_stream_read_probe(bufs[i % copies].data_ptr(), CEILING_BYTES, sink.data_ptr(),
                                                       wg)
                if rc:
                    abi.check(rc, "aljabr_rocm_stream_read_probe")
            for i in range(launches):
                go(i)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            head_start(torch)
            start.record(stream)
            for i in range(launches):
                go(i)
            end.record(stream)
            end.synchronize()
            us = start.elapsed_time(end) * 1e3 / launches
            gbs = CEILING_BYTES / us / 1e3
            out["by_workgroups"][str(wg)] = {"us": round(us, 3), "GBs": round(gbs, 1),
                                             "frac": round(gbs / HBM_PEAK_GBS, 4)}
            if best is None or us < best[1]:
                best = (wg, us, gbs)
    out.update(best_workgroups=best[0], us=round(best[1], 3), GBs=round(best[2], 1),
               frac=round(best[2] / HBM_PEAK_GBS, 4))
    del bufs
    torch.cuda.empty_cache()
    return out


def copy_probe(torch, stream) -> None:
    """A plain device copy of known size, for calibrating the HBM counters."""
    n = 64 << 20                                   # 64 Mi floats = 256 MiB each way
    a = torch.randn(n, device="cuda:0")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": 4 * n, "launches": 20}), flush=True)


def decode_bench(abi, torch, stream, batch: int, ctx: int, steps: int, make_model, cfg):
    """make_model(max_batch, max_seq) -> DeviceLlama."""
    max_seq = ctx + 2 * steps + 8
    model = make_model(batch, max_seq)
    # Context of `ctx` tokens: fill the fp16 KV cache with N(0,1) values.
    kp, vp = model.kv_cache_ptrs()
    total = model.kv_cache_elems()
    chunk = 1 << 26
    g = torch.Generator(device="cuda:0").manual_seed(77)
    for base_ptr in (kp, vp):
        off = 0
        while off < total:
            n = min(chunk, total - off)
            r = torch.randn(n, generator=g, device="cuda:0").half()
            torch.cuda.synchronize()
            abi.call("aljabr_rocm_memcpy_d2d", base_ptr + 2 * off, r.data_ptr(), 2 * n)
            abi.call("aljabr_rocm_synchronize")
            off += n
            del r
    tok = torch.randint(0, cfg["vocab"], (batch,), dtype=torch.int32, device="cuda:0",
                        generator=torch.Generator(device="cuda:0").manual_seed(5))
    torch.cuda.synchronize()
    def timed(step_fn, first_pos):
        nonlocal tok
        with torch.cuda.stream(stream):
            pos = torch.full((batch,), first_pos, dtype=torch.int32, device="cuda:0")
            tok = step_fn(tok, pos, batch)           # warm-up step (captures the graph)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            positions = [torch.full((batch,), first_pos + 1 + i, dtype=torch.int32, device="cuda:0")
                         for i in range(steps)]
            torch.cuda.synchronize()
            head_start(torch)
            start.record(stream)
            for i in range(steps):
                tok = step_fn(tok, positions[i], batch)
            end.record(stream)
            end.synchronize()
        return start.elapsed_time(end) / steps

    # Every step appends one row per sequence, so the two timings cover
    # contexts ctx .. ctx + steps and ctx + steps + 1 .. ctx + 2 steps + 1.
    ms_eager = timed(model.decode, ctx)
    ms = timed(model.decode_graph, ctx + steps + 1)
    # Per-kernel roofline breakdown: one more step with a HIP event after every
    # launch group (device time per group; the events themselves add a little).
    with torch.cuda.stream(stream):
        pos = torch.full((batch,), ctx + 2 * steps + 2, dtype=torch.int32, device="cuda:0")
        _, groups = model.decode_profile(tok, pos, batch)
    model.close()
    prof_us = sum(g["us"] for g in groups)
    kernels = []
    for g in sorted(groups, key=lambda g: -g["us"]):
        gbs = g["bytes"] / g["us"] / 1e3 if g["us"] > 0 else 0.0
        kernels.append({"group": g["name"], "launches": g["launches"], "us": round(g["us"], 1),
                        "share": round(g["us"] / prof_us, 3), "bytes": int(g["bytes"]), "GBs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 3)})
    return {"batch": batch, "context": ctx, "ms_per_step": round(ms, 3), "tokens_per_s": round(batch * 1000.0 / ms, 1),
            "path": "captured HIP graph of the whole step",
            "ms_per_step_eager": round(ms_eager, 3), "tokens_per_s_eager": round(batch * 1000.0 / ms_eager, 1),
            "profiled_ms": round(prof_us / 1e3, 3), "kernels": kernels}


def host_weights(torch, weights: dict) -> dict:
    """Device weights (random_weights layout) as the oracle's numpy arrays."""
    import numpy as np

    def get(t):
        a = t.cpu().numpy()
        return a.view(np.uint16) if t.dtype == torch.float16 else a
    return {k: [get(t) for t in v] if isinstance(v, list) else get(v) for k, v in weights.items()}


def decode_runs(args, abi, torch, stream, keep_host: bool = False):
    """random-init Llama-3-8B-shaped NF4 decode at batch
    1 and 32, context 2048. With keep_host also returns the weights as host
    arrays (the CPU baseline's oracle decode runs on the same model)."""
    from aljabr_amd.llama import LLAMA3_8B, DeviceLlama, random_weights
    log("building random-init Llama-3-8B-shaped NF4 model")
    t0 = time.perf_counter()
    weights = random_weights(LLAMA3_8B, seed=1)
    log(f"model built in {time.perf_counter() - t0:.1f} s")
    dec = []
    for batch in (1, 32):
        log(f"decode batch {batch}, context 2048")
        dec.append(decode_bench(abi, torch, stream, batch, 2048, args.decode_steps,
                                lambda b, s: DeviceLlama(LLAMA3_8B, weights, max_batch=b, max_seq=s), LLAMA3_8B))
    host = host_weights(torch, weights) if keep_host else None
    del weights
    torch.cuda.empty_cache()
    return (dec, host) if keep_host else dec


# GGUF Q4_K_M layout of a Llama-3-8B file: Q4_K projections and embedding,
# Q6_K attn_v, ffn_down and output.
Q4_K_M = dict(tok_embed=12, wq=12, wk=12, wv=14, wo=12, w_gate=12, w_up=12, w_down=14, lm_head=14)


def gguf_weights(torch, cfg: dict, types: dict, seed: int = 3) -> dict:
    """Synthetic typed weights on the device for DeviceLlama.typed (random
    K-quant codes with fp16 block scales ~1/256, fp32 norms near 1)."""
    from aljabr_amd.llama import PROJ, proj_shapes
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    shapes = proj_shapes(cfg)
    w = {k: [] for k in PROJ}
    w["attn_norm"], w["ffn_norm"] = [], []
    for _ in range(cfg["layers"]):
        for name in PROJ:
            n, k = shapes[name]
            w[name].append((types[name], kquant_blocks(torch, types[name], n, k, g)))
        w["attn_norm"].append(1.0 + 0.1 * torch.randn(cfg["dim"], generator=g, device="cuda:0"))
        w["ffn_norm"].append(1.0 + 0.1 * torch.randn(cfg["dim"], generator=g, device="cuda:0"))
    w["out_norm"] = 1.0 + 0.1 * torch.randn(cfg["dim"], generator=g, device="cuda:0")
    w["tok_embed"] = (types["tok_embed"], kquant_blocks(torch, types["tok_embed"], cfg["vocab"], cfg["dim"], g))
    w["lm_head"] = (types["lm_head"], kquant_blocks(torch, types["lm_head"], cfg["vocab"], cfg["dim"], g))
    torch.cuda.synchronize()
    return w


def gguf_decode_runs(args, abi, torch, stream):
    """The GGUF runner path: a Llama-3-8B-shaped Q4_K_M session (typed
    weights) decoding at batch 1 and 32, context 2048."""
    from aljabr_amd.llama import LLAMA3_8B, DeviceLlama
    log("building synthetic Llama-3-8B-shaped Q4_K_M model")
    weights = gguf_weights(torch, LLAMA3_8B, Q4_K_M)
    dec = []
    for batch in (1, 32):
        log(f"GGUF Q4_K_M decode batch {batch}, context 2048")
        r = decode_bench(abi, torch, stream, batch, 2048, args.decode_steps,
                         lambda b, s: DeviceLlama.typed(LLAMA3_8B, weights, max_batch=b, max_seq=s), LLAMA3_8B)
        r["weights"] = "GGUF Q4_K_M layout (Q4_K; Q6_K attn_v, ffn_down, output), synthetic codes"
        dec.append(r)
    del weights
    torch.cuda.empty_cache()
    return dec


def registered_step_runs(args, abi, torch, stream, ctx: int = 2048):
    """The Metal ABI's registered whole step (init_kv_cache, register_*,
    decode_step_token) at the Llama-3-8B Q4_K_M shapes, batch 1, context
    `ctx`: device weights, fp32 position-major KV caches prefilled with
    N(0,1) rows through sync_kv_cache, SiLU FFN. Each call returns the greedy
    token, so the time per token includes the call's own wait and host work
    (wall clock), as the Java runner sees it."""
    import ctypes
    from aljabr_amd.llama import LLAMA3_8B
    cfg = LLAMA3_8B
    lib = abi.load()
    log("registered whole step: Llama-3-8B Q4_K_M, batch 1")
    w = gguf_weights(torch, cfg, Q4_K_M, seed=11)
    L, dim, ffn = cfg["layers"], cfg["dim"], cfg["ffn"]
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    steps = max(args.decode_steps, 10)
    max_seq = ctx + steps + 8
    abi.call("aljabr_rocm_reset_decode_state")
    strides = (ctypes.c_int * L)(*([nkv * hd] * L))
    abi.call("aljabr_rocm_init_kv_cache", L, max_seq, strides)
    g = torch.Generator(device="cuda:0").manual_seed(21)
    prefix = torch.randn(ctx * nkv * hd, generator=g, device="cuda:0")
    torch.cuda.synchronize()
    for l in range(L):
        abi.call("aljabr_rocm_sync_kv_cache", l, ctx, prefix.data_ptr(), prefix.data_ptr())
    del prefix
    attn_norm = torch.cat(w["attn_norm"]).contiguous()
    ffn_norm = torch.cat(w["ffn_norm"]).contiguous()
    torch.cuda.synchronize()
    abi.call("aljabr_rocm_register_norm_buffer", 3, attn_norm.data_ptr(), attn_norm.numel() * 4)
    abi.call("aljabr_rocm_register_norm_buffer", 1, ffn_norm.data_ptr(), ffn_norm.numel() * 4)
    for l in range(L):
        t = {k: w[k][l] for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")}
        abi.call("aljabr_rocm_register_decode_layer", l, l,
                 *[t[k][1].data_ptr() for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")],
                 *[t[k][0] for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")],
                 nh * hd, nkv * hd, nkv * hd, nh * hd, dim, ffn, nh, nkv, hd, nkv * hd, cfg["rope_base"], 0,
                 1.0, 0.0, 0, 0, 0, 0, 0)
    abi.call("aljabr_rocm_register_output", w["out_norm"].data_ptr(), w["lm_head"][1].data_ptr(), w["lm_head"][0],
             dim, cfg["vocab"], 0.0)
    abi.call("aljabr_rocm_register_token_embd", w["tok_embed"][1].data_ptr(), w["tok_embed"][0], dim, 1.0)
    abi.call("aljabr_rocm_set_decode_activation", 1)
    torch.cuda.synchronize()
    tok = 17
    for i in range(3):                              # warm-up positions ctx .. ctx+2
        tok = lib.aljabr_rocm_decode_step_token(ctx + i, 0, cfg["eps"], tok, None)
        if tok < 0:
            abi.check(tok, "aljabr_rocm_decode_step_token")
    t0 = time.perf_counter()
    for i in range(steps):
        tok = lib.aljabr_rocm_decode_step_token(ctx + 3 + i, 0, cfg["eps"], tok, None)
        if tok < 0:
            abi.check(tok, "aljabr_rocm_decode_step_token")
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    abi.call("aljabr_rocm_reset_decode_state")
    del w, attn_norm, ffn_norm
    torch.cuda.empty_cache()
    return {"batch": 1, "context": ctx, "ms_per_token": round(ms, 3), "tokens_per_s": round(1000.0 / ms, 1),
            "weights": "GGUF Q4_K_M layout (Q4_K; Q6_K attn_v, ffn_down, output), synthetic codes",
            "kv_cache": "fp32 [max_seq][n_kv*head_dim] per layer (the Metal step's layout)",
            "timing": "wall clock per decode_step_token call (each waits for its step and returns the token)"}


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(no multi-GPU path: every box has one MI355X).", file=sys.stderr)
        sys.exit(2)
    import torch
    from aljabr_amd import abi
    abi.init(0)
    # One stream for torch (memory plumbing) and the C ABI, so their work is
    # ordered and the HIP events below time the kernels' own stream.
    stream = torch.cuda.Stream()
    abi.call("aljabr_rocm_set_stream", stream.cuda_stream)
    abi.call("aljabr_rocm_set_sync_mode", 0)
    with torch.cuda.stream(stream):
        if args.copy_probe:
            copy_probe(torch, stream)
        elif args.decode_only:
            print(json.dumps({"decode": decode_runs(args, abi, torch, stream)}), flush=True)
        elif args.kquant_only:
            print(json.dumps({"gguf_q4_0_q8_0": gguf_q_bench(abi, torch, stream),
                              "gguf_kquant": kquant_bench(abi, torch, stream)}), flush=True)
        elif args.small_m_only:
            ms = tuple(int(v) for v in args.small_m.split(","))
            print(json.dumps({"small_m_gemm": small_m_bench(abi, torch, stream, ms=ms)}), flush=True)
        elif args.prefill_only:
            print(json.dumps({"prefill_attention": prefill_bench(abi, torch, stream)}), flush=True)
        elif args.attention_only:
            print(json.dumps({"attention": attention_bench(abi, torch, stream)}), flush=True)
        elif args.step_only:
            print(json.dumps({"registered_step": registered_step_runs(args, abi, torch, stream)}), flush=True)
        elif args.stream_ceiling:
            wgs = (args.ceiling_workgroups,) if args.ceiling_workgroups > 0 else (256, 512, 1024, 2048, 4096, 8192)
            print(json.dumps({"stream_ceiling": stream_ceiling(abi, torch, stream, wgs=wgs)}), flush=True)
        elif args.gguf_decode_only:
            print(json.dumps({"decode_gguf_q4_k_m": gguf_decode_runs(args, abi, torch, stream)}), flush=True)
        else:
            run(args, abi, torch, stream)


def run(args, abi, torch, stream) -> None:
    step_bytes = nf4_bytes(FFN, K_MODEL) * 2 + nf4_bytes(K_MODEL, FFN)
    copies = args.copies or max(2, -(-512_000_000 // step_bytes))
    log(f"building {copies} NF4 MLP weight copies ({copies * step_bytes / 1e6:.0f} MB)")
    mats = make_mlp_copies(abi, torch, copies)
    log(f"timing {args.steps} steps after >= {args.clock_warmup_ms:.0f} ms of clock warm-up and {args.warmup} "
        "warmup steps")
    ms, clock_ms, clock_steps, idle_ms = time_mlp(abi, torch, stream, mats, args.steps, args.warmup,
                                                  args.clock_warmup_ms, idle_start=True)
    launches = 3 * args.steps
    per_launch_ms = ms / launches
    gbs = step_bytes * args.steps / (ms / 1e3) / 1e9
    per_launch_bytes = nf4_bytes(FFN, K_MODEL)   # all three launches move 33,030,144 + x + y bytes
    achieved = per_launch_bytes / (per_launch_ms / 1e3) / 1e9
    del mats
    torch.cuda.empty_cache()
    log("stream ceiling: plain reads of the same 33 MB")
    ceiling = stream_ceiling(abi, torch, stream)

    result = {
        "metric": "NF4 matvec HBM GB/s (% peak) + Llama-3-8B-shape NF4 decode tokens/s, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_ms": round(clock_ms, 1),
        "clock_warmup_steps": clock_steps,
        "ms_per_step": round(ms / args.steps, 5),
        "timed_region": f"{args.steps} steps after a synchronize and a ~0.4 ms GPU spin queued ahead of the start "
                        "event (the launches are enqueued while the GPU spins; the spin is not timed)",
        "idle_start": {"ms_per_step": round(idle_ms / args.steps, 5),
                       "avg_launch_us": round(idle_ms / (3 * args.steps) * 1e3, 3),
                       "note": "the same region started on an idle GPU (no spin): it also times the host's "
                               "enqueue of the first launches"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: NF4 weights quantized on device from N(0,0.02), x ~ N(0,1), "
                f"{copies} rotating weight copies ({copies * step_bytes / 1e6:.0f} MB)",
        "config": {"workload": "nf4_mlp_matvec_llama3_8b_batch1",
                   "shapes": ["14336x4096", "14336x4096", "4096x14336"], "nf4_block": BLOCK,
                   "weights": "nf4 codes + fp32 absmax", "activations": "f32",
                   "batch": 1, "parallelism": "none (1 GPU)"},
        "pct_peak_hbm": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_record(KERNEL),
                     "kernel": KERNEL, "bytes_per_launch": per_launch_bytes,
                     "avg_launch_us": round(per_launch_ms * 1e3, 3),
                     "stream_ceiling_us": ceiling["us"], "stream_ceiling_frac": ceiling["frac"]},
    }
    tail = {}
    # A memory-bound section leaves the GPU measurably slower for a second or
    # so (measured: Q4_0 14336x4096 at M = 1 8.7 us, 9.6 us right after the
    # attention grid, 8.8 us after a 2 s pause), so every later section starts
    # after an idle pause and then runs its own untimed warm-up launches.
    result["section_pause_s"] = args.section_pause_s

    def pause():
        torch.cuda.synchronize()
        time.sleep(args.section_pause_s)

    if not args.no_extra:
        log("small-M NF4 GEMM (M = 1, 4, 16, 32, 64)")
        pause()
        tail["small_m_gemm"] = small_m_bench(abi, torch, stream)
        log("GQA decode attention")
        pause()
        tail["attention"] = attention_bench(abi, torch, stream)
        log("GGUF Q4_0 / Q8_0 matvec (M = 1, 8)")
        pause()
        tail["gguf_q4_0_q8_0"] = gguf_q_bench(abi, torch, stream)
        log("GGUF K-quant matvec (Q4_K, Q6_K; M = 1, 4, 8)")
        pause()
        result["gguf_kquant"] = kquant_bench(abi, torch, stream)
        log("prefill attention (T = S = 512, 2048, 8192)")
        pause()
        result["prefill_attention"] = prefill_bench(abi, torch, stream)

    llama_host = None
    if not args.no_decode:
        pause()
        result["decode"], llama_host = decode_runs(args, abi, torch, stream, keep_host=not args.no_cpu)
        pause()
        result["decode_gguf_q4_k_m"] = gguf_decode_runs(args, abi, torch, stream)
        pause()
        result["registered_step"] = registered_step_runs(args, abi, torch, stream)

    result["stream_ceiling"] = {k: ceiling[k] for k in ("bytes_per_launch", "best_workgroups", "us", "GBs", "frac")}
    if not args.no_cpu:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds, llama_host)
    del llama_host
    # The configs[0], [1] and [3] figures close the line.
    result.update(tail)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
