// matvec_nf4.hip - batch-1 NF4 matvec, K split across the waves of a
// workgroup, T rows per workgroup pipelined in straight-line code.
//
// Layout recap: codes u8 [N*K/2], byte j = (code[2j] << 4) | code[2j+1];
// absmax fp32 per 2^k >= 32 elements of the flat [N,K] index
// (STC/DequantizationKernel.java:84-102).
//
// Why this shape (measured on MI355X): with a 16-entry fp32 codebook in LDS
// most lookups of a wave hit the same few banks, which LDS serves as
// broadcasts; a lane reading 128 contiguous activation bytes per row costs the
// address unit 64 cache lines per instruction, so activations are staged
// once per wave with coalesced loads through LDS; and the compiler drains
// every outstanding load at a loop back-edge, so the T rows of a workgroup
// are unrolled, with the loads of row t+PF issued before row t is computed.
//
// Workgroup = S waves (S = K/2048); wave w owns K chunk w (32 weights,
// 16 code bytes, per lane) for rows [row0, row0+T). Codebook lookups read the
// fp32 level from LDS byte address nibble*4: one shift and one mask per four
// nibbles pre-scale them, one v_bfe_u32 extracts each address. After T rows
// one butterfly reduces all T row sums across the wave, and the S wave
// partials of each row meet in LDS once.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kChunk = 2048;
constexpr int kMaxWaves = 8;

template <int OFF>
__device__ __forceinline__ uint32_t ubfe8(uint32_t v) {
    uint32_t r;
    asm("v_bfe_u32 %0, %1, %2, 8" : "=v"(r) : "v"(v), "i"(OFF));
    return r;
}

// 32 weights (one 16-byte code word) against the lane's 32 activations.
__device__ __forceinline__ float nf4_word_dot(u32x4 q, const float (&xv)[32], const char *lut) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t hi4 = (w[i] >> 2) & 0x3C3C3C3Cu;   // even elements (high nibbles) * 4
        const uint32_t lo4 = (w[i] << 2) & 0x3C3C3C3Cu;   // odd elements (low nibbles) * 4
        float vh[4], vl[4];
        vh[0] = *reinterpret_cast<const float *>(lut + ubfe8<0>(hi4));
        vh[1] = *reinterpret_cast<const float *>(lut + ubfe8<8>(hi4));
        vh[2] = *reinterpret_cast<const float *>(lut + ubfe8<16>(hi4));
        vh[3] = *reinterpret_cast<const float *>(lut + ubfe8<24>(hi4));
        vl[0] = *reinterpret_cast<const float *>(lut + ubfe8<0>(lo4));
        vl[1] = *reinterpret_cast<const float *>(lut + ubfe8<8>(lo4));
        vl[2] = *reinterpret_cast<const float *>(lut + ubfe8<16>(lo4));
        vl[3] = *reinterpret_cast<const float *>(lut + ubfe8<24>(lo4));
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            p0 = fmaf(vh[t], xv[8 * i + 2 * t], p0);
            p1 = fmaf(vl[t], xv[8 * i + 2 * t + 1], p1);
        }
    }
    return p0 + p1;
}

template <int T, int PF>
__global__ __launch_bounds__(kMaxWaves * 64) void nf4_rows_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                                  const uint8_t *__restrict__ codes,
                                                                  const float *__restrict__ absmax, int N, int K,
                                                                  int bs_shift) {
    static_assert(T <= 16 && PF >= 1, "tile shape");
    __shared__ float lut_f[16];
    __shared__ float part[kMaxWaves][16];
    extern __shared__ float4 xstage[];           // 512 float4 (8 KiB) per wave
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    const int row0 = blockIdx.x * T;
    const int k0 = wave * kChunk + lane * 32;    // K % 2048 == 0: every lane is in range
    const size_t row_bytes = static_cast<size_t>(K) >> 1;

    // Activations: lane L needs floats [32L, 32L+32) of the wave's chunk.
    // Coalesced float4 loads (float4 f = 64j + lane) are transposed through
    // the wave's LDS window; float4 f is stored at slot (f/8)*8 + ((f%8) ^
    // ((f/8)%8)), so both the stores and the 8 ds_read_b128 per lane are
    // bank-conflict free. Activation loads go out first: vmcnt retires in
    // order, so waiting for them leaves the weight loads below in flight.
    const float4 *xw = reinterpret_cast<const float4 *>(x + wave * kChunk);
    float4 xl[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xl[j] = xw[64 * j + lane];

    // Per-row load addresses; rows past N re-read row N-1 (results dropped).
    // Everything below is branch-free so the loads stay in issue order.
    const uint8_t *qp = codes + (k0 >> 1);
    u32x4 q[T];
    float sc[T];
#pragma unroll
    for (int t = 0; t < PF && t < T; ++t) {
        const int row = min(row0 + t, N - 1);
        q[t] = load_stream16(qp + row * row_bytes);
        sc[t] = absmax[(static_cast<size_t>(row) * K + k0) >> bs_shift];
    }

    const float level = nf4_level_sel(threadIdx.x & 15);
    if (threadIdx.x < 16) lut_f[threadIdx.x] = level;
    float4 *win = xstage + wave * 512;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int f = 64 * j + lane;
        win[(f >> 3) * 8 + ((f & 7) ^ ((f >> 3) & 7))] = xl[j];
    }
    __syncthreads();
    float xv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = win[lane * 8 + (i ^ (lane & 7))];
        xv[4 * i + 0] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
    }
    const char *lut = reinterpret_cast<const char *>(lut_f);

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t + PF < T) {
            const int row = min(row0 + t + PF, N - 1);
            q[t + PF] = load_stream16(qp + row * row_bytes);
            sc[t + PF] = absmax[(static_cast<size_t>(row) * K + k0) >> bs_shift];
        }
        acc[t] = nf4_word_dot(q[t], xv, lut) * sc[t];
        // Keep the written pipeline: without these the compiler defers every
        // row's arithmetic to the end and holds all lookups in registers.
        asm volatile("" : "+v"(acc[t]));
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tot = wave_sum_rows<T>(acc);
    if (lane < T) part[wave][wave_rows_index<T>(lane)] = tot;
    __syncthreads();
    if (threadIdx.x < T && row0 + static_cast<int>(threadIdx.x) < N) {
        float v = 0.0f;
        for (int w = 0; w < S; ++w) v += part[w][threadIdx.x];
        y[row0 + threadIdx.x] = v;
    }
}

}  // namespace

// Rows per workgroup T: the largest of {16, 8, 4, 2} that still leaves ~12
// waves per CU.
int enqueue_nf4_rows(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift) {
    const int S = (K + kChunk - 1) / kChunk;
    if (K % kChunk != 0 || S > kMaxWaves || bs_shift < 5 || !aligned(Bq, 16) || !aligned(A, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    int T = 2;
    for (int cand = 16; cand >= 2; cand >>= 1)
        if (static_cast<long long>((N + cand - 1) / cand) * S >= 12LL * cus) {
            T = cand;
            break;
        }
    hipStream_t s = current_stream();
    const dim3 grid((N + T - 1) / T), block(64 * S);
    const size_t lds = static_cast<size_t>(S) * 512 * sizeof(float4);
    switch (T) {
    case 16: hipLaunchKernelGGL((nf4_rows_kernel<16, 4>), grid, block, lds, s, C, A, Bq, absmax, N, K, bs_shift); break;
    case 8: hipLaunchKernelGGL((nf4_rows_kernel<8, 4>), grid, block, lds, s, C, A, Bq, absmax, N, K, bs_shift); break;
    case 4: hipLaunchKernelGGL((nf4_rows_kernel<4, 4>), grid, block, lds, s, C, A, Bq, absmax, N, K, bs_shift); break;
    default: hipLaunchKernelGGL((nf4_rows_kernel<2, 2>), grid, block, lds, s, C, A, Bq, absmax, N, K, bs_shift); break;
    }
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
