// codec.hip - bit-exact decoders and device-side encoders for NF4, GGUF Q4_0,
// GGUF Q8_0 and fp16, plus a byte fill kernel.
//
// Decoders reproduce the reference's fp32 results bit for bit:
//   NF4  STC/DequantizationKernel.java:84-102     T[nibble] * absmax[(2j)/bs]
//   Q4_0 GRT/GgufBlockDequantizer.java:33-37,403-416  (q-8)*d + 0.0f  (+0.0f turns -0 into +0)
//   Q8_0 GRT/GgufBlockDequantizer.java:231-265    (int8)q * d
//   Q4_K GRT/GgufKBlockDequantizer.java:32-90      (d*sc)*q - dmin*min (0 for a zero min code or dmin == 0)
//   Q6_K GRT/GgufKBlockDequantizer.java:320-425    (d*scale)*(q6-32)
//   F16  GRT/GgufQuantTables.java:143-165         (canonical NaN)
// Encoders reproduce GWR/GGUFWriter.java:163-209,360-387 bit for bit (fp32
// scale for quantizing, writer-rounded fp16 scale stored, Java Math.round).
// Every multiply uses __fmul_rn so the compiler cannot contract it.
#include "dequant.hpp"
#include "device.hpp"
#include "internal.hpp"

namespace aljabr {
namespace {

constexpr int kThreads = 256;

inline unsigned blocks_for(long long n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

// One thread per packed byte (two elements).
__global__ __launch_bounds__(kThreads) void nf4_dequant_kernel(float *__restrict__ dst, const uint8_t *__restrict__ codes,
                                                               const float *__restrict__ absmax, long long numel,
                                                               int bs) {
    const long long j = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    const long long bytes = (numel + 1) / 2;
    if (j >= bytes) return;
    const uint8_t b = codes[j];
    const float s = absmax[(2 * j) / bs];
    dst[2 * j] = __fmul_rn(nf4_level(b >> 4), s);
    if (2 * j + 1 < numel) dst[2 * j + 1] = __fmul_rn(nf4_level(b & 15), s);
}

// One thread per 32-element block.
__global__ __launch_bounds__(kThreads) void q4_0_dequant_kernel(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                                                long long nblocks) {
    const long long blk = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (blk < nblocks) dq_q4_0_block(src + blk * 18, dst + blk * 32);
}

__global__ __launch_bounds__(kThreads) void q8_0_dequant_kernel(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                                                long long nblocks) {
    const long long blk = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (blk < nblocks) dq_q8_0_block(src + blk * 34, dst + blk * 32);
}

// One thread per 32-element sub-block of a Q4_K super-block.
__global__ __launch_bounds__(kThreads) void q4_k_dequant_kernel(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                                                long long nsub) {
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (t < nsub) dq_q4_k_sub(src + (t >> 3) * 144, static_cast<int>(t & 7), dst + (t << 5));
}

// One thread per 16-element scale group of a Q6_K super-block.
__global__ __launch_bounds__(kThreads) void q6_k_dequant_kernel(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                                                long long ngroups) {
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (t < ngroups) dq_q6_k_group(src + (t >> 4) * 210, static_cast<int>(t & 15), dst + (t << 4));
}

__global__ __launch_bounds__(kThreads) void f16_dequant_kernel(float *__restrict__ dst, const uint16_t *__restrict__ src,
                                                               long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) dst[i] = f16_bits_to_f32_exact(src[i]);
}

__device__ __forceinline__ float block_max_abs(const float *v, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float a = fabsf(v[i]);
        m = a > m ? a : m;   // Math.max(m, |v|) for non-NaN data
    }
    return m;
}

// GWR/GGUFWriter.java:179-194
__global__ __launch_bounds__(kThreads) void q4_0_quant_kernel(uint8_t *__restrict__ dst, const float *__restrict__ src,
                                                              long long nblocks) {
    const long long blk = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (blk >= nblocks) return;
    const float *v = src + blk * 32;
    uint8_t *o = dst + blk * 18;
    const float scale = __fdiv_rn(block_max_abs(v, 32), 7.0f);
    const uint32_t h = f32_to_f16_writer(scale);
    o[0] = static_cast<uint8_t>(h & 0xff);
    o[1] = static_cast<uint8_t>(h >> 8);
    for (int i = 0; i < 16; ++i) {
        const int lo = scale == 0.0f ? 0 : min(max(java_round(__fdiv_rn(v[i], scale)), -8), 7);
        const int hi = scale == 0.0f ? 0 : min(max(java_round(__fdiv_rn(v[16 + i], scale)), -8), 7);
        o[2 + i] = static_cast<uint8_t>(((hi + 8) << 4) | (lo + 8));
    }
}

// GWR/GGUFWriter.java:163-177
__global__ __launch_bounds__(kThreads) void q8_0_quant_kernel(uint8_t *__restrict__ dst, const float *__restrict__ src,
                                                              long long nblocks) {
    const long long blk = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (blk >= nblocks) return;
    const float *v = src + blk * 32;
    uint8_t *o = dst + blk * 34;
    const float scale = __fdiv_rn(block_max_abs(v, 32), 127.0f);
    const uint32_t h = f32_to_f16_writer(scale);
    o[0] = static_cast<uint8_t>(h & 0xff);
    o[1] = static_cast<uint8_t>(h >> 8);
    for (int i = 0; i < 32; ++i) {
        const int q = scale == 0.0f ? 0 : java_round(__fdiv_rn(v[i], scale));
        o[2 + i] = static_cast<uint8_t>(min(max(q, -127), 127) & 0xff);
    }
}

// NF4 encoder (build-defined; the reference's quantizer is absent): absmax per
// block, then the nearest codebook level of v/absmax, exact midpoints to the
// lower level. One thread per block; blocks of an odd-sized tail are partial.
__global__ __launch_bounds__(kThreads) void nf4_quant_kernel(uint8_t *__restrict__ codes, float *__restrict__ absmax,
                                                             const float *__restrict__ src, long long numel, int bs) {
    const long long g = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    const long long groups = (numel + bs - 1) / bs;
    if (g >= groups) return;
    const long long begin = g * bs;
    const long long end = begin + bs < numel ? begin + bs : numel;
    float m = 0.0f;
    for (long long i = begin; i < end; ++i) {
        const float a = fabsf(src[i]);
        m = a > m ? a : m;
    }
    absmax[g] = m;
    // bs is even, so every byte of this block belongs to it alone.
    for (long long i = begin; i < end; i += 2) {
        uint32_t pair = 0;
        for (int h = 0; h < 2 && i + h < end; ++h) {
            int c = 7;
            if (m != 0.0f) {
                const float v = __fdiv_rn(src[i + h], m);
                c = 15;
                for (int k = 0; k < 15; ++k) {
                    const float mid = __fmul_rn(__fadd_rn(nf4_level(k), nf4_level(k + 1)), 0.5f);
                    if (v <= mid) {
                        c = k;
                        break;
                    }
                }
            }
            pair |= static_cast<uint32_t>(c) << (h == 0 ? 4 : 0);
        }
        codes[i >> 1] = static_cast<uint8_t>(pair);
    }
}

// GWR/GGUFWriter.java:155-161 (encodeF16)
__global__ __launch_bounds__(kThreads) void f16_quant_kernel(uint16_t *__restrict__ dst, const float *__restrict__ src,
                                                             long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) dst[i] = static_cast<uint16_t>(f32_to_f16_writer(src[i]));
}

__global__ __launch_bounds__(kThreads) void fill_u8_kernel(uint8_t *__restrict__ dst, uint8_t value, long long n) {
    long long i = (static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x) * 16;
    if (i + 16 <= n && (reinterpret_cast<uintptr_t>(dst + i) & 15) == 0) {
        const uint32_t w = value * 0x01010101u;
        *reinterpret_cast<uint4 *>(dst + i) = make_uint4(w, w, w, w);
        return;
    }
    for (long long k = i; k < n && k < i + 16; ++k) dst[k] = value;
}

}  // namespace
}  // namespace aljabr

using namespace aljabr;

extern "C" {

int aljabr_rocm_dequantize(void *dst_f32, const void *src, const void *absmax, long long numel, int type,
                           int blockSize) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(dst_f32 && src, "dst and src must be non-null device pointers");
    ALJ_REQUIRE(numel >= 0, "numel must be non-negative");
    if (numel == 0) return ALJABR_ROCM_OK;
    hipStream_t s = current_stream();
    float *dst = static_cast<float *>(dst_f32);
    const uint8_t *in = static_cast<const uint8_t *>(src);
    switch (type) {
    case ALJABR_ROCM_TYPE_NF4:
        ALJ_REQUIRE(absmax, "NF4 needs absmax");
        ALJ_REQUIRE(blockSize > 0 && blockSize % 2 == 0, "NF4 blockSize must be positive and even");
        hipLaunchKernelGGL(nf4_dequant_kernel, dim3(blocks_for((numel + 1) / 2)), dim3(kThreads), 0, s, dst, in,
                           static_cast<const float *>(absmax), numel, blockSize);
        break;
    case ALJABR_ROCM_TYPE_Q4_0:
        ALJ_REQUIRE(numel % 32 == 0, "Q4_0 numel must be a multiple of 32");
        hipLaunchKernelGGL(q4_0_dequant_kernel, dim3(blocks_for(numel / 32)), dim3(kThreads), 0, s, dst, in,
                           numel / 32);
        break;
    case ALJABR_ROCM_TYPE_Q8_0:
        ALJ_REQUIRE(numel % 32 == 0, "Q8_0 numel must be a multiple of 32");
        hipLaunchKernelGGL(q8_0_dequant_kernel, dim3(blocks_for(numel / 32)), dim3(kThreads), 0, s, dst, in,
                           numel / 32);
        break;
    case ALJABR_ROCM_TYPE_Q4_K:
        ALJ_REQUIRE(numel % 256 == 0, "Q4_K numel must be a multiple of 256");
        hipLaunchKernelGGL(q4_k_dequant_kernel, dim3(blocks_for(numel / 32)), dim3(kThreads), 0, s, dst, in,
                           numel / 32);
        break;
    case ALJABR_ROCM_TYPE_Q6_K:
        ALJ_REQUIRE(numel % 256 == 0, "Q6_K numel must be a multiple of 256");
        hipLaunchKernelGGL(q6_k_dequant_kernel, dim3(blocks_for(numel / 16)), dim3(kThreads), 0, s, dst, in,
                           numel / 16);
        break;
    case ALJABR_ROCM_TYPE_F16:
        hipLaunchKernelGGL(f16_dequant_kernel, dim3(blocks_for(numel)), dim3(kThreads), 0, s, dst,
                           static_cast<const uint16_t *>(src), numel);
        break;
    default:
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "dequantize: unsupported type %d", type);
    }
    return finish_launch("dequantize");
}

int aljabr_rocm_quantize(void *dst, void *absmax_out, const void *src_f32, long long numel, int type, int blockSize) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(dst && src_f32, "dst and src must be non-null device pointers");
    ALJ_REQUIRE(numel >= 0, "numel must be non-negative");
    if (numel == 0) return ALJABR_ROCM_OK;
    hipStream_t s = current_stream();
    const float *in = static_cast<const float *>(src_f32);
    switch (type) {
    case ALJABR_ROCM_TYPE_NF4: {
        ALJ_REQUIRE(absmax_out, "NF4 needs an absmax output");
        ALJ_REQUIRE(blockSize > 0 && blockSize % 2 == 0, "NF4 blockSize must be positive and even");
        const long long groups = (numel + blockSize - 1) / blockSize;
        hipLaunchKernelGGL(nf4_quant_kernel, dim3(blocks_for(groups)), dim3(kThreads), 0, s,
                           static_cast<uint8_t *>(dst), static_cast<float *>(absmax_out), in, numel, blockSize);
        break;
    }
    case ALJABR_ROCM_TYPE_Q4_0:
        ALJ_REQUIRE(numel % 32 == 0, "Q4_0 tensors must be divisible by 32 elements");
        hipLaunchKernelGGL(q4_0_quant_kernel, dim3(blocks_for(numel / 32)), dim3(kThreads), 0, s,
                           static_cast<uint8_t *>(dst), in, numel / 32);
        break;
    case ALJABR_ROCM_TYPE_Q8_0:
        ALJ_REQUIRE(numel % 32 == 0, "Q8_0 tensors must be divisible by 32 elements");
        hipLaunchKernelGGL(q8_0_quant_kernel, dim3(blocks_for(numel / 32)), dim3(kThreads), 0, s,
                           static_cast<uint8_t *>(dst), in, numel / 32);
        break;
    case ALJABR_ROCM_TYPE_F16:
        hipLaunchKernelGGL(f16_quant_kernel, dim3(blocks_for(numel)), dim3(kThreads), 0, s,
                           static_cast<uint16_t *>(dst), in, numel);
        break;
    default:
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "quantize: unsupported type %d", type);
    }
    return finish_launch("quantize");
}

int aljabr_rocm_fill_u8(void *device_dst, int value, size_t bytes) {
    ALJ_CHECK_READY();
    if (bytes == 0) return ALJABR_ROCM_OK;
    ALJ_REQUIRE(device_dst, "dst must be a non-null device pointer");
    const long long n = static_cast<long long>(bytes);
    hipLaunchKernelGGL(fill_u8_kernel, dim3(blocks_for((n + 15) / 16)), dim3(kThreads), 0, current_stream(),
                       static_cast<uint8_t *>(device_dst), static_cast<uint8_t>(value & 0xff), n);
    return finish_launch("fill_u8");
}

}  // extern "C"
