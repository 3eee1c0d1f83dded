"""MI355X (gfx950) implementation of Aljabr's quantized-inference hot path.

The product is the C-ABI library ``libaljabr_rocm.so`` (HIP kernels for NF4 /
GGUF Q4_0 / Q8_0 / Q4_K / Q6_K dequant-fused matvec and small-M GEMM, split-K
GQA decode attention and device-resident decode steps) declared in
``include/aljabr_rocm.h``. ``aljabr_amd.abi`` binds it with ctypes,
``aljabr_amd.llama`` wraps the Llama decode session, and ``aljabr_amd/host``
holds the C++ mirror of the reference's ComputeProvider / ProviderSession /
ComputeBackend interface (``libaljabr_rocm_spi.so``).
"""
from . import abi  # noqa: F401

__all__ = ["abi"]
