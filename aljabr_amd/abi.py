"""ctypes binding of the C ABI in ``include/aljabr_rocm.h``.

This module is the Python counterpart of the FFM downcall table a Java provider
builds (MetalBinding's ``Linker.nativeLinker().downcallHandle`` table,
backend/metal/aljabr-backend-metal/.../binding/MetalBinding.java:1799-1818):
one declared signature per exported symbol and a status check that turns a
non-zero return into an exception carrying ``aljabr_rocm_last_error()``.

It loads ``libaljabr_rocm.so`` from this package directory and raises if the
library is missing: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaljabr_rocm.so")

OK = 0
ERR_NOT_INITIALIZED = -1
ERR_BAD_ARGUMENT = -2
ERR_UNSUPPORTED = -3
ERR_BUFFER = -4
ERR_DEVICE = -5

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_NF4 = 100

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_LL = ctypes.c_longlong
_SZ = ctypes.c_size_t


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("total_bytes", ctypes.c_uint64),
        ("free_bytes", ctypes.c_uint64),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width", ctypes.c_int32),
        ("l2_bytes", ctypes.c_int32),
        ("runtime_version", ctypes.c_int32),
        ("driver_version", ctypes.c_int32),
    ]


class LlamaConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "layers", "dim", "ffn", "n_heads", "n_kv_heads", "head_dim", "vocab", "max_seq",
        "nf4_block", "max_batch")] + [("rope_base", ctypes.c_float), ("eps", ctypes.c_float)]


_PP = ctypes.POINTER(ctypes.c_void_p)


class LlamaWeights(ctypes.Structure):
    _fields_ = [
        ("tok_embed", _P),
        ("attn_norm", _PP), ("ffn_norm", _PP),
        ("wq", _PP), ("wk", _PP), ("wv", _PP), ("wo", _PP),
        ("wq_absmax", _PP), ("wk_absmax", _PP), ("wv_absmax", _PP), ("wo_absmax", _PP),
        ("w_gate", _PP), ("w_up", _PP), ("w_down", _PP),
        ("w_gate_absmax", _PP), ("w_up_absmax", _PP), ("w_down_absmax", _PP),
        ("out_norm", _P),
        ("lm_head", _P),
    ]


class Tensor(ctypes.Structure):
    """aljabr_rocm_tensor: device data, type id, and (NF4) absmax and block size."""
    _fields_ = [("data", _P), ("absmax", _P), ("type", ctypes.c_int32), ("block_size", ctypes.c_int32)]


_TP = ctypes.POINTER(Tensor)


class LlamaTensors(ctypes.Structure):
    """aljabr_rocm_llama_tensors: a typed session's weights."""
    _fields_ = [
        ("tok_embed", Tensor),
        ("attn_norm", _PP), ("ffn_norm", _PP),
        ("wq", _TP), ("wk", _TP), ("wv", _TP), ("wo", _TP),
        ("w_gate", _TP), ("w_up", _TP), ("w_down", _TP),
        ("out_norm", _P),
        ("lm_head", Tensor),
    ]


# name -> (restype, argtypes); every symbol declared in include/aljabr_rocm.h.
class KernelStat(ctypes.Structure):
    """aljabr_rocm_kernel_stat: one launch group of a profiled decode step."""
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_int32), ("us", ctypes.c_double),
                ("bytes", ctypes.c_double)]


SIGNATURES = {
    "aljabr_rocm_init": (_I, [_I]),
    "aljabr_rocm_shutdown": (_I, []),
    "aljabr_rocm_is_initialized": (_I, []),
    "aljabr_rocm_device_count": (_I, [ctypes.POINTER(_I)]),
    "aljabr_rocm_device_info_get": (_I, [_I, ctypes.POINTER(DeviceInfo)]),
    "aljabr_rocm_last_error": (ctypes.c_char_p, []),
    "aljabr_rocm_version": (_I, []),
    "aljabr_rocm_set_stream": (_I, [_P]),
    "aljabr_rocm_get_stream": (_I, [ctypes.POINTER(_P)]),
    "aljabr_rocm_stream_scratch_bytes": (_I, [ctypes.POINTER(ctypes.c_size_t)]),
    "aljabr_rocm_stream_read_probe": (_I, [_P, ctypes.c_size_t, _P, _I]),
    "aljabr_rocm_set_sync_mode": (_I, [_I]),
    "aljabr_rocm_synchronize": (_I, []),
    "aljabr_rocm_alloc": (_I, [_SZ, ctypes.POINTER(_P)]),
    "aljabr_rocm_free": (_I, [_P]),
    "aljabr_rocm_memcpy_h2d": (_I, [_P, _P, _SZ]),
    "aljabr_rocm_memcpy_d2h": (_I, [_P, _P, _SZ]),
    "aljabr_rocm_memcpy_d2d": (_I, [_P, _P, _SZ]),
    "aljabr_rocm_fill_u8": (_I, [_P, _I, _SZ]),
    "aljabr_rocm_matvec_tb_nf4": (_I, [_P, _P, _P, _P, _I, _I, _I]),
    "aljabr_rocm_matvec_tb_q4_0": (_I, [_P, _P, _P, _I, _I]),
    "aljabr_rocm_matvec_tb_q8_0": (_I, [_P, _P, _P, _I, _I]),
    "aljabr_rocm_matvec_tb_half": (_I, [_P, _P, _P, _I, _I]),
    "aljabr_rocm_matvec_tb_q4_k": (_I, [_P, _P, _P, _I, _I]),
    "aljabr_rocm_matvec_tb_q6_k": (_I, [_P, _P, _P, _I, _I]),
    "aljabr_rocm_matvec_tb_q4_k_softcap": (_I, [_P, _P, _P, _I, _I, ctypes.c_float]),
    "aljabr_rocm_matvec_tb_q6_k_softcap": (_I, [_P, _P, _P, _I, _I, ctypes.c_float]),
    "aljabr_rocm_matvec_tb_batch": (_I, [_P, _P, _P, _I, _I, _I, _I]),
    "aljabr_rocm_matvec_tb_batch_nf4": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "aljabr_rocm_dequantize": (_I, [_P, _P, _P, _LL, _I, _I]),
    "aljabr_rocm_quantize": (_I, [_P, _P, _P, _LL, _I, _I]),
    "aljabr_rocm_attention_gqa": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I]),
    "aljabr_rocm_attention_gqa_noalloc": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I]),
    "aljabr_rocm_matvec_tb_pair": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "aljabr_rocm_matvec_tb_triple": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]),
    "aljabr_rocm_matvec_tb_triple_batch": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I]),
    "aljabr_rocm_ffn_gated_fused": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "aljabr_rocm_ffn_gated_fused_batch": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]),
    "aljabr_rocm_safetensors_open": (_I, [ctypes.c_char_p, _P]),
    "aljabr_rocm_safetensors_close": (_I, [_P]),
    "aljabr_rocm_safetensors_tensor_count": (_I, [_P, _P]),
    "aljabr_rocm_safetensors_find_tensor": (_I, [_P, ctypes.c_char_p, _P]),
    "aljabr_rocm_safetensors_tensor_info": (_I, [_P, ctypes.c_int64, _P, _I, _P, _P, _P, _P]),
    "aljabr_rocm_safetensors_tensor_data": (_I, [_P, ctypes.c_int64, _P]),
    "aljabr_rocm_safetensors_meta": (_I, [_P, ctypes.c_char_p, _P, _I]),
    "aljabr_rocm_safetensors_upload_nf4": (_I, [_P, ctypes.c_char_p, _P, _P, _P, _P, _P]),
    "aljabr_rocm_llama_create_safetensors": (_I, [ctypes.c_char_p, _P, _P]),
    "aljabr_rocm_fa4_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _I, _F]),
    "aljabr_rocm_fa4_attention_windowed": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _F, _I]),
    "aljabr_rocm_fa4_sdpa_available": (_I, []),
    "aljabr_rocm_fa4_bf16_available": (_I, []),
    "aljabr_rocm_paged_attention": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _F]),
    "aljabr_rocm_paged_attention_windowed": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _I,
                                                  _I, _F]),
    "aljabr_rocm_paged_attention_gqa": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _F]),
    "aljabr_rocm_paged_attention_gqa_windowed": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I,
                                                      _I, _I, _F]),
    "aljabr_rocm_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F]),
    "aljabr_rocm_rope": (_I, [_P, _P, _I, _I, _I, _F]),
    "aljabr_rocm_swiglu": (_I, [_P, _P, _P, _LL]),
    "aljabr_rocm_add_inplace": (_I, [_P, _P, _LL]),
    "aljabr_rocm_argmax": (_I, [_P, _P, _I, _I]),
    "aljabr_rocm_llama_create": (_I, [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights),
                                      ctypes.POINTER(_P)]),
    "aljabr_rocm_llama_create_typed": (_I, [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaTensors),
                                            ctypes.POINTER(_P)]),
    "aljabr_rocm_llama_create_gguf": (_I, [ctypes.c_char_p, _I, _I, ctypes.POINTER(_P)]),
    "aljabr_rocm_llama_config_get": (_I, [_P, ctypes.POINTER(LlamaConfig)]),
    "aljabr_rocm_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "aljabr_rocm_gguf_close": (_I, [_P]),
    "aljabr_rocm_gguf_tensor_count": (_I, [_P, ctypes.POINTER(ctypes.c_int64)]),
    "aljabr_rocm_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "aljabr_rocm_gguf_tensor_info": (_I, [_P, ctypes.c_int64, ctypes.c_char_p, _I, ctypes.POINTER(ctypes.c_int32),
                                          ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "aljabr_rocm_gguf_tensor_data": (_I, [_P, ctypes.c_int64, ctypes.POINTER(_P)]),
    "aljabr_rocm_gguf_meta_int": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "aljabr_rocm_gguf_meta_float": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "aljabr_rocm_gguf_meta_string": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p, _I]),
    "aljabr_rocm_llama_destroy": (_I, [_P]),
    "aljabr_rocm_llama_decode": (_I, [_P, _P, _P, _I, _P, _P]),
    "aljabr_rocm_llama_decode_graph": (_I, [_P, _P, _P, _I, _P, _P]),
    "aljabr_rocm_llama_decode_profile": (_I, [_P, _P, _P, _I, _P, _P, ctypes.POINTER(KernelStat), _I,
                                              ctypes.POINTER(_I)]),
    "aljabr_rocm_llama_hidden": (_I, [_P, ctypes.POINTER(_P)]),
    "aljabr_rocm_llama_kv_cache": (_I, [_P, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "aljabr_rocm_init_kv_cache": (_I, [_I, _I, _P]),
    "aljabr_rocm_sync_kv_cache": (_I, [_I, _I, _P, _P]),
    "aljabr_rocm_register_norm_buffer": (_I, [_I, _P, _SZ]),
    "aljabr_rocm_register_rope_freqs": (_I, [_I, _P, _I]),
    "aljabr_rocm_register_decode_layer": (_I, [_I, _I] + [_P] * 7 + [_I] * 7 + [_I] * 10 + [_F, _I, _F, _F]
                                          + [_I] * 5),
    "aljabr_rocm_register_output": (_I, [_P, _P, _I, _I, _I, _F]),
    "aljabr_rocm_register_token_embd": (_I, [_P, _I, _I, _F]),
    "aljabr_rocm_decode_step": (_I, [_I, _I, _F, _P, _P]),
    "aljabr_rocm_decode_step_token": (_I, [_I, _I, _F, _I, _P]),
    "aljabr_rocm_set_decode_activation": (_I, [_I]),
    "aljabr_rocm_reset_decode_state": (_I, []),
    "aljabr_rocm_wo_ffn_next_qkv_fused": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, _P, _P, _I, _F, _F, _P, _P, _P,
                                               _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I,
                                               _I, _I, _I]),
    "aljabr_rocm_wo_ffn_fused": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, _I, _P, _I, _P, _I, _I, _F, _P, _P, _P,
                                      _I, _I, _I, _I, _I]),
    "aljabr_rocm_wo_ffn_logits_fused": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, _P, _P, _I, _F, _F, _P, _P, _P,
                                             _I, _I, _I, _I, _I, _P, _P, _I, _I, _I, _P, _F]),
    "aljabr_rocm_wo_ffn_reset_x": (None, []),
    "aljabr_rocm_wo_ffn_fused_layer_batch": (_I, [_P, _P, _I, _I, _F, _I]),
}


class RocmError(RuntimeError):
    """A non-zero status from the C ABI, with the library's message."""

    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where} returned {status}: {message}")
        self.status = status
        self.where = where


_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library; raises FileNotFoundError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: build it with `python -m aljabr_amd.build` "
            "(there is no fallback implementation)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().aljabr_rocm_last_error()
    return msg.decode() if msg else ""


def check(status: int, where: str = "aljabr_rocm") -> None:
    if status != OK:
        raise RocmError(status, where, last_error())


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise RocmError on a non-zero status."""
    check(getattr(load(), name)(*args), name)


def device_count() -> int:
    n = _I(0)
    check(load().aljabr_rocm_device_count(ctypes.byref(n)), "aljabr_rocm_device_count")
    return n.value


def device_info(ordinal: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    check(load().aljabr_rocm_device_info_get(ordinal, ctypes.byref(info)), "aljabr_rocm_device_info_get")
    return info


def init(ordinal: int = 0) -> None:
    call("aljabr_rocm_init", ordinal)
