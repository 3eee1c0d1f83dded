// matvec_stream.hip - persistent, double-buffered batch-1 matvec for GGUF
// Q4_0 / Q8_0 rows whose K is not a multiple of 2048 (K <= 16384).
//
// A workgroup has S = ceil(K/2048) waves; wave w owns K chunk w for the whole
// launch, so its 32 activations per lane are loaded once and stay in VGPRs.
// Workgroups stride over groups of R rows (group g, g + gridDim.x, ...). While
// a wave dequantizes and accumulates group g, the loads of its next group are
// already in flight (two register buffers), which keeps HBM busy during the
// VALU work. Per group the S wave partials meet in LDS (double-buffered by
// iteration parity, one barrier per group) and R threads write y.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kMaxWaves = 8;

// ---------------------------------------------------------------------------
// GGUF Q4_0 / Q8_0: lane owns one 32-element block of its wave's chunk.
// ---------------------------------------------------------------------------
template <int NDW>
__device__ __forceinline__ void gguf_block(const uint8_t *blk, uint32_t (&q)[NDW], float &d) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(blk + 2);
    const uint32_t off = static_cast<uint32_t>(a & 3u);
    const uint32_t *p = reinterpret_cast<const uint32_t *>(a - off);
    uint32_t dw[NDW + 1];
#pragma unroll
    for (int i = 0; i < NDW; ++i) dw[i] = __builtin_nontemporal_load(p + i);
    uint32_t dbits;
    if (off) {
        dw[NDW] = *reinterpret_cast<const uint16_t *>(blk + 2 + 4 * NDW - 2);
        dbits = dw[0] & 0xffffu;
    } else {
        dw[NDW] = 0;
        dbits = *reinterpret_cast<const uint16_t *>(blk);
    }
    const uint32_t sh = off * 8u;
#pragma unroll
    for (int i = 0; i < NDW; ++i) q[i] = funnel_shift_right(dw[i + 1], dw[i], sh);
    d = f16_bits_to_f32(dbits);
}

template <int R, bool Q8>
struct GgufBuf {
    uint32_t q[R][Q8 ? 8 : 4];
    float d[R];
};

template <int R, bool Q8>
__device__ __forceinline__ void gguf_load(GgufBuf<R, Q8> &b, const uint8_t *__restrict__ w, int row0, int N, int nblk,
                                          int blk, bool active) {
    constexpr int BYTES = Q8 ? 34 : 18;
    if (!active) return;
    const size_t row_bytes = static_cast<size_t>(nblk) * BYTES;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, N - 1);
        gguf_block<Q8 ? 8 : 4>(w + row * row_bytes + static_cast<size_t>(blk) * BYTES, b.q[r], b.d[r]);
    }
}

template <int R, bool Q8>
__device__ __forceinline__ void gguf_dot(const GgufBuf<R, Q8> &b, const float (&xv)[32], float xs, float (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float p0 = 0.0f, p1 = 0.0f;
        if constexpr (!Q8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = b.q[r][i] & 0x0F0F0F0Fu;          // elements 4i..4i+3
                const uint32_t hi = (b.q[r][i] >> 4) & 0x0F0F0F0Fu;   // elements 16+4i..
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    p0 = fmaf(static_cast<float>((lo >> (8 * t)) & 0xffu), xv[4 * i + t], p0);
                    p1 = fmaf(static_cast<float>((hi >> (8 * t)) & 0xffu), xv[16 + 4 * i + t], p1);
                }
            }
            acc[r] = b.d[r] * fmaf(-8.0f, xs, p0 + p1);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = b.q[r][i] ^ 0x80808080u;               // int8 -> uint8 + 128
                p0 = fmaf(static_cast<float>(u & 0xffu), xv[4 * i + 0], p0);
                p1 = fmaf(static_cast<float>((u >> 8) & 0xffu), xv[4 * i + 1], p1);
                p0 = fmaf(static_cast<float>((u >> 16) & 0xffu), xv[4 * i + 2], p0);
                p1 = fmaf(static_cast<float>(u >> 24), xv[4 * i + 3], p1);
            }
            acc[r] = b.d[r] * fmaf(-128.0f, xs, p0 + p1);
        }
    }
}

template <int R>
struct GgufSmem {
    float part[2][kMaxWaves][R];
};

template <int R>
__device__ __forceinline__ void publish_g(GgufSmem<R> &sm, float (&acc)[R], int parity, int wave, int lane, int S,
                                          float *__restrict__ y, int row0, int N) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[r]);
        if (lane == 0) sm.part[parity][wave][r] = v;
    }
    __syncthreads();
    if (threadIdx.x < R) {
        float v = 0.0f;
        for (int w = 0; w < S; ++w) v += sm.part[parity][w][threadIdx.x];
        if (row0 + static_cast<int>(threadIdx.x) < N) y[row0 + threadIdx.x] = v;
    }
}

template <int R, bool Q8>
__global__ __launch_bounds__(kMaxWaves * 64) void gguf_stream_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                                     const uint8_t *__restrict__ w, int N, int K) {
    __shared__ GgufSmem<R> sm;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    const int nblk = K >> 5;
    const int blk = wave * 64 + lane;
    const bool active = blk < nblk;
    float xv[32];
    float xs = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) xv[i] = 0.0f;
    if (active) {
        const float4 *xp = reinterpret_cast<const float4 *>(x + blk * 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 t = xp[i];
            xv[4 * i + 0] = t.x;
            xv[4 * i + 1] = t.y;
            xv[4 * i + 2] = t.z;
            xv[4 * i + 3] = t.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            s0 += xv[i];
            s1 += xv[16 + i];
        }
        xs = s0 + s1;
    }
    const int groups = (N + R - 1) / R;
    GgufBuf<R, Q8> a, b;
    float acc[R];
    int g = blockIdx.x;
    int parity = 0;
    if (g < groups) gguf_load<R, Q8>(a, w, g * R, N, nblk, blk, active);
    while (g < groups) {
        const int g1 = g + gridDim.x;
        if (g1 < groups) gguf_load<R, Q8>(b, w, g1 * R, N, nblk, blk, active);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if (active) gguf_dot<R, Q8>(a, xv, xs, acc);
        publish_g<R>(sm, acc, parity, wave, lane, S, y, g * R, N);
        parity ^= 1;
        if (g1 >= groups) break;
        const int g2 = g1 + gridDim.x;
        if (g2 < groups) gguf_load<R, Q8>(a, w, g2 * R, N, nblk, blk, active);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if (active) gguf_dot<R, Q8>(b, xv, xs, acc);
        publish_g<R>(sm, acc, parity, wave, lane, S, y, g1 * R, N);
        parity ^= 1;
        g = g2;
    }
}

// Launch shape: R rows per group, about 16 resident waves per CU.
struct StreamShape {
    int R, grid, S;
};

StreamShape stream_shape(int N, int S) {
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    StreamShape sh{};
    sh.S = S;
    sh.R = 4;
    const int per_cu = (16 + S - 1) / S;
    const int groups = (N + sh.R - 1) / sh.R;
    long long grid = static_cast<long long>(cus) * per_cu;
    sh.grid = static_cast<int>(grid < groups ? grid : groups);
    return sh;
}

}  // namespace

int enqueue_gguf_stream(float *C, const float *A, const uint8_t *B, int K, int N, int type) {
    const int nchunks = (K / 32 + 63) / 64;
    if ((type != ALJABR_ROCM_TYPE_Q4_0 && type != ALJABR_ROCM_TYPE_Q8_0) || K % 32 != 0 || nchunks > kMaxWaves ||
        !aligned(A, 16) || !aligned(B, 4))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    const StreamShape sh = stream_shape(N, nchunks);
    hipStream_t s = current_stream();
    const dim3 grid(sh.grid), block(64 * sh.S);
    const bool q8 = type == ALJABR_ROCM_TYPE_Q8_0;
#define ALJ_GS(RR)                                                                                          \
    do {                                                                                                    \
        if (q8) hipLaunchKernelGGL((gguf_stream_kernel<RR, true>), grid, block, 0, s, C, A, B, N, K);       \
        else hipLaunchKernelGGL((gguf_stream_kernel<RR, false>), grid, block, 0, s, C, A, B, N, K);         \
    } while (0)
    ALJ_GS(4);
#undef ALJ_GS
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
