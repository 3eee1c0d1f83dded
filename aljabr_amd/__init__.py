"""MI355X (gfx950) implementation of Aljabr's quantized-inference hot path.

The product is the C-ABI library ``libaljabr_rocm.so`` (HIP kernels for NF4 /
GGUF Q4_0 / Q8_0 dequant-fused matvec and small-M GEMM, split-K GQA decode
attention and a device-resident Llama decode step) declared in
``include/aljabr_rocm.h``. ``aljabr_amd.abi`` binds it with ctypes and
``aljabr_amd.provider`` mirrors the reference's ComputeProvider /
ProviderSession / ComputeBackend interface on top of it.
"""
from . import abi  # noqa: F401

__all__ = ["abi"]
