// matvec_stream.hip - persistent, double-buffered batch-1 matvec (NF4, GGUF
// Q4_0, GGUF Q8_0) for K <= 16384.
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

constexpr int kChunk = 2048;
constexpr int kMaxWaves = 8;

template <int OFF>
__device__ __forceinline__ uint32_t ubfe8(uint32_t v) {
    uint32_t r;
    asm("v_bfe_u32 %0, %1, %2, 8" : "=v"(r) : "v"(v), "i"(OFF));
    return r;
}

template <int R>
struct StreamSmem {
    float lut[16];                      // must stay the first member (LDS offset 0)
    float part[2][kMaxWaves][R];
};

template <int R>
struct NF4Buf {
    u32x4 q[R];
    float s[R];
};

template <int R>
__device__ __forceinline__ void nf4_load(NF4Buf<R> &b, const uint8_t *__restrict__ codes,
                                         const float *__restrict__ absmax, int row0, int N, int K, int k0,
                                         int bs_shift, bool active) {
    if (!active) return;
    const size_t row_bytes = static_cast<size_t>(K) >> 1;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, N - 1);
        b.q[r] = load_stream16(codes + row * row_bytes + (k0 >> 1));
        b.s[r] = absmax[(static_cast<size_t>(row) * K + k0) >> bs_shift];
    }
}

template <int R>
__device__ __forceinline__ void nf4_dot(const NF4Buf<R> &b, const float (&xv)[32], const char *lut, float (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t w[4] = {b.q[r].x, b.q[r].y, b.q[r].z, b.q[r].w};
        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t hi4 = (w[i] >> 2) & 0x3C3C3C3Cu;   // even elements (high nibbles) * 4
            const uint32_t lo4 = (w[i] << 2) & 0x3C3C3C3Cu;   // odd elements (low nibbles) * 4
            p0 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<0>(hi4)), xv[8 * i + 0], p0);
            p1 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<0>(lo4)), xv[8 * i + 1], p1);
            p0 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<8>(hi4)), xv[8 * i + 2], p0);
            p1 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<8>(lo4)), xv[8 * i + 3], p1);
            p0 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<16>(hi4)), xv[8 * i + 4], p0);
            p1 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<16>(lo4)), xv[8 * i + 5], p1);
            p0 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<24>(hi4)), xv[8 * i + 6], p0);
            p1 = fmaf(*reinterpret_cast<const float *>(lut + ubfe8<24>(lo4)), xv[8 * i + 7], p1);
        }
        acc[r] = (p0 + p1) * b.s[r];
    }
}

// Sum the S wave partials of a group and write the R outputs.
template <int R>
__device__ __forceinline__ void publish(StreamSmem<R> &sm, float (&acc)[R], int parity, int wave, int lane, int S,
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

template <int R>
__global__ __launch_bounds__(kMaxWaves * 64) void nf4_stream_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                                    const uint8_t *__restrict__ codes,
                                                                    const float *__restrict__ absmax, int N, int K,
                                                                    int bs_shift) {
    __shared__ StreamSmem<R> sm;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    if (threadIdx.x < 16) sm.lut[threadIdx.x] = nf4_level(threadIdx.x);
    const int k0 = wave * kChunk + lane * 32;
    const bool active = k0 < K;                   // lanes past K (last chunk) contribute 0
    float xv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) xv[i] = 0.0f;
    if (active) {
        const float4 *xp = reinterpret_cast<const float4 *>(x + k0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 t = xp[i];
            xv[4 * i + 0] = t.x;
            xv[4 * i + 1] = t.y;
            xv[4 * i + 2] = t.z;
            xv[4 * i + 3] = t.w;
        }
    }
    __syncthreads();
    const char *lut = reinterpret_cast<const char *>(sm.lut);
    const int groups = (N + R - 1) / R;
    NF4Buf<R> a, b;
    float acc[R];
    int g = blockIdx.x;
    int parity = 0;
    if (g < groups) nf4_load<R>(a, codes, absmax, g * R, N, K, k0, bs_shift, active);
    // Two groups per trip so the buffers swap roles without register copies.
    while (g < groups) {
        const int g1 = g + gridDim.x;
        if (g1 < groups) nf4_load<R>(b, codes, absmax, g1 * R, N, K, k0, bs_shift, active);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if (active) nf4_dot<R>(a, xv, lut, acc);
        publish<R>(sm, acc, parity, wave, lane, S, y, g * R, N);
        parity ^= 1;
        if (g1 >= groups) break;
        const int g2 = g1 + gridDim.x;
        if (g2 < groups) nf4_load<R>(a, codes, absmax, g2 * R, N, K, k0, bs_shift, active);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        if (active) nf4_dot<R>(b, xv, lut, acc);
        publish<R>(sm, acc, parity, wave, lane, S, y, g1 * R, N);
        parity ^= 1;
        g = g2;
    }
}

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

// Launch shape: rows per group and workgroups, tunable from the environment
// (ALJABR_ROCM_STREAM_R, ALJABR_ROCM_STREAM_WG_PER_CU) for sweeps.
int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

struct StreamShape {
    int R, grid, S;
};

StreamShape stream_shape(int N, int S) {
    static const int env_r = env_int("ALJABR_ROCM_STREAM_R", 4);
    static const int env_per_cu = env_int("ALJABR_ROCM_STREAM_WG_PER_CU", 0);
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    StreamShape sh{};
    sh.S = S;
    sh.R = env_r;
    if (sh.R != 1 && sh.R != 2 && sh.R != 4 && sh.R != 8) sh.R = 4;
    // Aim at ~16 resident waves per CU.
    int per_cu = env_per_cu;
    if (per_cu <= 0) per_cu = (16 + S - 1) / S;
    const int groups = (N + sh.R - 1) / sh.R;
    long long grid = static_cast<long long>(cus) * per_cu;
    sh.grid = static_cast<int>(grid < groups ? grid : groups);
    return sh;
}

}  // namespace

int enqueue_nf4_stream(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift) {
    const int nchunks = (K + kChunk - 1) / kChunk;
    if (K % 32 != 0 || nchunks > kMaxWaves || bs_shift < 5 || !aligned(Bq, 16) || !aligned(A, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    const StreamShape sh = stream_shape(N, nchunks);
    hipStream_t s = current_stream();
    const dim3 grid(sh.grid), block(64 * sh.S);
    switch (sh.R) {
    case 1: hipLaunchKernelGGL(nf4_stream_kernel<1>, grid, block, 0, s, C, A, Bq, absmax, N, K, bs_shift); break;
    case 2: hipLaunchKernelGGL(nf4_stream_kernel<2>, grid, block, 0, s, C, A, Bq, absmax, N, K, bs_shift); break;
    case 8: hipLaunchKernelGGL(nf4_stream_kernel<8>, grid, block, 0, s, C, A, Bq, absmax, N, K, bs_shift); break;
    default: hipLaunchKernelGGL(nf4_stream_kernel<4>, grid, block, 0, s, C, A, Bq, absmax, N, K, bs_shift); break;
    }
    return ALJABR_ROCM_OK;
}

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
    switch (sh.R) {
    case 1: ALJ_GS(1); break;
    case 2: ALJ_GS(2); break;
    case 8: ALJ_GS(8); break;
    default: ALJ_GS(4); break;
    }
#undef ALJ_GS
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
