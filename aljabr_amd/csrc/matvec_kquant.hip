// matvec_kquant.hip - GGUF Q4_K / Q6_K matvec and small-M GEMM for any K that
// is a whole number of 256-weight super-blocks, and the output soft cap of the
// *_softcap entry points.
//
// Y[m][n] = sum_k X[m][k] * W[n][k] with W rows of K/256 super-blocks
// (layouts in kquant.hpp). One wave per row: lane l takes lane j = l % 8 of
// super-blocks l/8, l/8 + 8, ...; the M token rows are read from L2 per
// super-block and the M sums reduced across the wave at the end of the row.
// The batch-1 fast path for K % 2048 == 0 is the rows kernel
// (matvec_rows.hip); this kernel covers the other shapes and M >= 2.
//
// Reference: GRT/GgufQ4RawDot.java:38-148, GRT/GgufQ6RawDot.java:33-133 (row
// dots), MTLC/aljabr_metal_matvec_api.h:48-55 and
// MTLC/aljabr_metal_matvec_api.m:428-505 (entry points, soft cap).
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"
#include "kquant.hpp"

namespace aljabr {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool Q6, int M>
__global__ __launch_bounds__(kThreads) void kquant_mv_kernel(float *__restrict__ C, const float *__restrict__ A,
                                                             const uint8_t *__restrict__ W, int N, int K) {
    constexpr int BB = Q6 ? kQ6KBytes : kQ4KBytes;
    constexpr int HI = Q6 ? kQ6KHigh : kQ4KHigh;
    const int lane = threadIdx.x & 63;
    const int j = lane & 7;
    const int lo = Q6 ? q6k_lo_elem(j) : q4k_lo_elem(j);
    const int nsb = K >> 8;
    const size_t row_bytes = static_cast<size_t>(nsb) * BB;
    const int first = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int stride = gridDim.x * kWavesPerBlock;
    for (int row = first; row < N; row += stride) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
        const uint8_t *r = W + static_cast<size_t>(row) * row_bytes;
        for (int sb = lane >> 3; sb < nsb; sb += 8) {
            const uint8_t *blk = r + static_cast<size_t>(sb) * BB;
            KScales s;
            Q4KWords w4;
            Q6KWords w6;
            if constexpr (Q6) {
                load_q6k(w6, blk, j);
                s = q6k_scales(w6, j);
            } else {
                load_q4k(w4, blk, j);
                s = q4k_scales(w4.hdr, j);
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float *x = A + static_cast<size_t>(m) * K + (sb << 8) + lo;
                float xlo[16], xhi[16];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f32x4 a = *reinterpret_cast<const f32x4 *>(x + 4 * i);
                    const f32x4 b = *reinterpret_cast<const f32x4 *>(x + HI + 4 * i);
                    xlo[4 * i] = a.x; xlo[4 * i + 1] = a.y; xlo[4 * i + 2] = a.z; xlo[4 * i + 3] = a.w;
                    xhi[4 * i] = b.x; xhi[4 * i + 1] = b.y; xhi[4 * i + 2] = b.z; xhi[4 * i + 3] = b.w;
                }
                float sxlo = 0.0f, sxhi = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    sxlo += xlo[i];
                    sxhi += xhi[i];
                }
                float plo, phi;
                if constexpr (Q6) q6k_dots(w6, j, xlo, xhi, plo, phi);
                else q4k_dots(w4.q, xlo, xhi, plo, phi);
                acc[m] += k_combine<Q6>(s, plo, phi, sxlo, sxhi);
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float v = wave_sum(acc[m]);
            if (lane == 0) C[static_cast<size_t>(m) * N + row] = v;
        }
    }
}

__global__ __launch_bounds__(kThreads) void softcap_kernel(float *__restrict__ y, long long n, float cap) {
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) y[i] = cap * static_cast<float>(tanh(static_cast<double>(y[i] / cap)));
}

template <bool Q6>
void launch_kquant_mv(float *C, const float *A, const uint8_t *W, int K, int N, int M, hipStream_t s) {
    const long long want = (static_cast<long long>(N) + kWavesPerBlock - 1) / kWavesPerBlock;
    const dim3 grid(static_cast<unsigned>(want < 65536 ? want : 65536)), block(kThreads);
    switch (M) {
    case 1: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 1>), grid, block, 0, s, C, A, W, N, K); break;
    case 2: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 2>), grid, block, 0, s, C, A, W, N, K); break;
    case 3: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 3>), grid, block, 0, s, C, A, W, N, K); break;
    case 4: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 4>), grid, block, 0, s, C, A, W, N, K); break;
    case 5: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 5>), grid, block, 0, s, C, A, W, N, K); break;
    case 6: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 6>), grid, block, 0, s, C, A, W, N, K); break;
    case 7: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 7>), grid, block, 0, s, C, A, W, N, K); break;
    default: hipLaunchKernelGGL((kquant_mv_kernel<Q6, 8>), grid, block, 0, s, C, A, W, N, K); break;
    }
}

}  // namespace

// C[M][N] = A[M][K] . W^T for Q4_K / Q6_K rows (K % 256 == 0, A and W 16-byte
// aligned); batch 1 with K % 2048 == 0 takes the rows kernel.
int enqueue_matmul_kquant(float *C, const float *A, const uint8_t *W, int K, int N, int type, int M, float *part,
                          size_t part_floats) {
    if ((type != ALJABR_ROCM_TYPE_Q4_K && type != ALJABR_ROCM_TYPE_Q6_K) || K % 256 != 0 || N < 1 || M < 1)
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (!aligned(A, 16) || !aligned(W, 16))
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "K-quant matvec needs A and B 16-byte aligned");
    if (M == 1 && enqueue_rows(C, A, W, nullptr, K, N, type, 0) == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
    hipStream_t s = current_stream();
    const bool q6 = type == ALJABR_ROCM_TYPE_Q6_K;
    int m0 = 0;
    if (M >= 2 && K % 512 == 0 && mfma_enabled()) {
        // Matrix cores, 32 tokens per pass; a last single token takes the rows kernel.
        while (M - m0 >= 2) {
            const int mm = M - m0 < 32 ? M - m0 : 32;
            const int rc = enqueue_kquant_mfma(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, W,
                                               K, N, type, mm, part, part_floats);
            if (rc != ALJABR_ROCM_OK) return rc;
            m0 += mm;
        }
        if (m0 < M && enqueue_rows(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, W, nullptr, K,
                                   N, type, 0) == ALJABR_ROCM_OK)
            return ALJABR_ROCM_OK;
    }
    for (; m0 < M; m0 += 8) {
        const int mm = M - m0 < 8 ? M - m0 : 8;
        float *c = C + static_cast<size_t>(m0) * N;
        const float *a = A + static_cast<size_t>(m0) * K;
        if (q6) launch_kquant_mv<true>(c, a, W, K, N, mm, s);
        else launch_kquant_mv<false>(c, a, W, K, N, mm, s);
    }
    return ALJABR_ROCM_OK;
}

int enqueue_softcap(float *y, long long n, float cap) {
    if (n <= 0) return ALJABR_ROCM_OK;
    hipLaunchKernelGGL(softcap_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       current_stream(), y, n, cap);
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
