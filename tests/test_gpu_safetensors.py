"""GPU parity of the safetensors NF4 path: Llama-family files with Hugging
Face names and NF4 projections in the safetensor engine's convention
(".qweight" U8 + ".scales" F32, group 128; AccelWeightBridge.java:184-222)
are loaded by aljabr_rocm_llama_create_safetensors and decoded on the device;
every step is compared with the oracle's typed decode over the same weights
(NF4 at block 128, BF16 tensors widened to fp32): logits within 1e-3
relative L2, greedy tokens equal up to near-ties. Also: one NF4 weight
uploaded by aljabr_rocm_safetensors_upload_nf4 drives the NF4 matvec, and
files the step cannot decode faithfully are refused."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import safetensors_writer as sw
from conftest import rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, dim=512, ffn=1536, n_heads=8, n_kv_heads=2, head_dim=64, vocab=1024, max_seq=16,
           rope_base=500000.0, eps=1e-5, nf4_block=128)
NF4 = 100


def _model(oracle, cfg, dense=(), lm_head="nf4", emb_dtype="BF16", seed=3):
    """(tensors for the writer, oracle weights). `dense` names the projections
    stored as BF16 .weight instead of NF4."""
    dim, ffn, nh, nkv, hd, vocab, L = (cfg[k] for k in ("dim", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab",
                                                         "layers"))
    qd, kvd = nh * hd, nkv * hd
    tensors, w = [], {k: [] for k in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")}
    s = seed * 1000

    def dense_entry(name, arr, dtype):
        if dtype == "BF16":
            bits = sw.bf16_bits(arr)
            tensors.append((name, "BF16", arr.shape, bits.tobytes()))
            return (0, sw.bf16_to_f32(bits).reshape(arr.shape))
        if dtype == "F16":
            h = arr.astype(np.float16)
            tensors.append((name, "F16", arr.shape, h.tobytes()))
            return (1, h.view(np.uint16))
        tensors.append((name, "F32", arr.shape, np.ascontiguousarray(arr, np.float32).tobytes()))
        return (0, np.ascontiguousarray(arr, np.float32))

    def nf4_entry(base, n, k, seed_):
        codes, absmax = oracle.nf4_quantize(oracle.normal(seed_, n * k, 0.0, 0.5 / np.sqrt(k)), 128)
        tensors.append((base + ".qweight", "U8", (n, k // 2), codes.tobytes()))
        tensors.append((base + ".scales", "F32", (n * k // 128,), absmax.astype(np.float32).tobytes()))
        return (NF4, codes, absmax)

    emb = oracle.normal(s, vocab * dim).reshape(vocab, dim).astype(np.float32)
    w["tok_embed"] = dense_entry("model.embed_tokens.weight", emb, emb_dtype)
    shapes = {"wq": ("self_attn.q_proj", qd, dim), "wk": ("self_attn.k_proj", kvd, dim),
              "wv": ("self_attn.v_proj", kvd, dim), "wo": ("self_attn.o_proj", dim, qd),
              "w_gate": ("mlp.gate_proj", ffn, dim), "w_up": ("mlp.up_proj", ffn, dim),
              "w_down": ("mlp.down_proj", dim, ffn)}
    for l in range(L):
        pre = f"model.layers.{l}."
        an = (1.0 + 0.1 * oracle.normal(s + 10 * l + 1, dim)).astype(np.float32)
        fn = (1.0 + 0.1 * oracle.normal(s + 10 * l + 2, dim)).astype(np.float32)
        w["attn_norm"].append(dense_entry(pre + "input_layernorm.weight", an, "BF16")[1])
        w["ffn_norm"].append(dense_entry(pre + "post_attention_layernorm.weight", fn, "F32")[1])
        for i, (key, (name, n, k)) in enumerate(shapes.items()):
            if key in dense:
                arr = (oracle.normal(s + 100 * l + 7 * i, n * k, 0.0, 0.5 / np.sqrt(k))).reshape(n, k)
                w[key].append(dense_entry(pre + name + ".weight", arr, "BF16"))
            else:
                w[key].append(nf4_entry(pre + name, n, k, s + 100 * l + 7 * i))
    on = (1.0 + 0.1 * oracle.normal(s + 7, dim)).astype(np.float32)
    w["out_norm"] = dense_entry("model.norm.weight", on, "F32")[1]
    if lm_head == "nf4":
        w["lm_head"] = nf4_entry("lm_head", vocab, dim, s + 9)
    elif lm_head == "f16":
        w["lm_head"] = dense_entry("lm_head.weight", oracle.normal(s + 9, vocab * dim, 0.0, 0.05).reshape(vocab, dim),
                                   "F16")
    else:
        w["lm_head"] = w["tok_embed"]
    return tensors, w


def _decode_against_oracle(dev, oracle, model, cfg, weights, batch, steps=5):
    import torch
    refs = [oracle.TypedLlamaOracle(cfg, weights) for _ in range(batch)]
    first = (np.array([5, 17, 901], np.int32) % cfg["vocab"])[:batch]
    start = np.array([0, 1, 3], np.int32)[:batch]
    logits = torch.empty(batch * cfg["vocab"], dtype=torch.float32, device="cuda:0")
    cur = first.copy()
    for step in range(steps):
        pos = np.maximum(0, step - start).astype(np.int32)
        cur = np.where(pos == 0, first, cur).astype(np.int32)
        nxt = model.decode(dev.put(cur), dev.put(pos), batch, logits=logits)
        got_tok = dev.get(nxt)
        got_logits = dev.get(logits).reshape(batch, -1)
        for b in range(batch):
            ref_tok, ref_logits, _ = refs[b].decode(int(cur[b]), int(pos[b]))
            assert np.isfinite(got_logits[b]).all(), (step, b)
            assert rel_l2(got_logits[b], ref_logits) <= 1e-3, (step, b)
            assert got_tok[b] == ref_tok or \
                ref_logits[ref_tok] - ref_logits[got_tok[b]] <= 1e-3 * np.abs(ref_logits).max()
            cur[b] = ref_tok


@pytest.mark.parametrize("variant,batch", [("all_nf4", 1), ("all_nf4", 3), ("mixed", 2), ("tied_f16", 1)])
def test_safetensors_decode_matches_oracle(rocm, dev, oracle, tmp_path, variant, batch):
    from aljabr_amd.llama import DeviceLlama
    if variant == "all_nf4":
        tensors, w = _model(oracle, CFG)
    elif variant == "mixed":
        tensors, w = _model(oracle, CFG, dense=("wv", "w_down"), lm_head="f16")
    else:
        tensors, w = _model(oracle, CFG, lm_head="tied", emb_dtype="F16")
    path = str(tmp_path / f"{variant}.safetensors")
    sw.write(path, tensors, {"format": "pt"})
    model = DeviceLlama.from_safetensors(path, CFG, max_batch=batch, max_seq=CFG["max_seq"])
    assert model.cfg["nf4_block"] == 128
    _decode_against_oracle(dev, oracle, model, CFG, w, batch)
    model.close()


def test_upload_nf4_drives_the_nf4_matvec(rocm, dev, oracle, tmp_path):
    n, k = 300, 2048
    codes, absmax = oracle.nf4_quantize(oracle.normal(77, n * k, 0.0, 0.02), 128)
    path = str(tmp_path / "one.safetensors")
    sw.write(path, [("w.qweight", "U8", (n, k // 2), codes.tobytes()),
                    ("w.scales", "F32", (n * k // 128,), absmax.astype(np.float32).tobytes())])
    lib = rocm.load()
    h = ctypes.c_void_p()
    rocm.check(lib.aljabr_rocm_safetensors_open(path.encode(), ctypes.byref(h)), "open")
    c, a = ctypes.c_void_p(), ctypes.c_void_p()
    rows, cols, blk = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
    rocm.check(lib.aljabr_rocm_safetensors_upload_nf4(h, b"w", ctypes.byref(c), ctypes.byref(a), ctypes.byref(rows),
                                                      ctypes.byref(cols), ctypes.byref(blk)), "upload_nf4")
    lib.aljabr_rocm_safetensors_close(h)
    assert (rows.value, cols.value, blk.value) == (n, k, 128)
    x = oracle.normal(78, k)
    xd, y = dev.put(x), dev.empty(n)
    rocm.call("aljabr_rocm_matvec_tb_nf4", dev.ptr(y), dev.ptr(xd), c.value, a.value, k, n, 128)
    assert rel_l2(dev.get(y), oracle.nf4_matvec(codes, absmax, x, n, k, 128)) <= 1e-3
    rocm.call("aljabr_rocm_free", c.value)
    rocm.call("aljabr_rocm_free", a.value)


@pytest.mark.parametrize("problem", ["q_norm", "f16_scales", "missing", "bad_shape"])
def test_safetensors_refusals(rocm, oracle, tmp_path, problem):
    from aljabr_amd import abi
    from aljabr_amd.llama import DeviceLlama
    tensors, _ = _model(oracle, CFG)
    want = abi.ERR_BAD_ARGUMENT
    if problem == "q_norm":
        tensors.append(("model.layers.0.self_attn.q_norm.weight", "F32", (64,), np.ones(64, np.float32).tobytes()))
        want = abi.ERR_UNSUPPORTED
    elif problem == "f16_scales":
        i = [t[0] for t in tensors].index("model.layers.1.mlp.up_proj.scales")
        name, _, shape, raw = tensors[i]
        tensors[i] = (name, "F16", shape, np.frombuffer(raw, np.float32).astype(np.float16).tobytes())
        want = abi.ERR_UNSUPPORTED
    elif problem == "missing":
        tensors = [t for t in tensors if not t[0].startswith("model.layers.1.mlp.down_proj")]
    else:
        i = [t[0] for t in tensors].index("model.norm.weight")
        tensors[i] = ("model.norm.weight", "F32", (256,), bytes(1024))
    path = str(tmp_path / f"{problem}.safetensors")
    sw.write(path, tensors)
    with pytest.raises(abi.RocmError) as e:
        DeviceLlama.from_safetensors(path, CFG, max_batch=1, max_seq=8)
    assert e.value.status == want
