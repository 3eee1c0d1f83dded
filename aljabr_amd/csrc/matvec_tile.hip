// matvec_tile.hip - batch-1/2 dequant-fused matvec, K split across the waves
// of a workgroup (NF4, GGUF Q4_0, GGUF Q8_0).
//
// Tile = R rows x one 2048-element K chunk (every lane owns 32 consecutive
// weights of the chunk: 16 packed NF4 bytes or one 18/34-byte GGUF block).
// A workgroup holds S <= 8 waves, one per chunk, and covers R whole rows; a
// wave walks its chunks c = wave, wave + S, ... . Per chunk a lane issues all
// R weight loads, its absmax/scale loads and its 32 activations at once (the
// activations are reused by the R rows, so they cost 8/R of the weight bytes
// in L1/L2 traffic), dequantizes in registers and accumulates per row. Wave
// partials are reduced with DPP, combined across the S waves through LDS and
// written once per row; no atomics, deterministic.
//
// NF4 codebook lookups read a 16-entry LDS table at byte address nibble*4; the
// nibbles of a packed dword are pre-scaled by four with one shift and one mask
// per four of them, and each address is then a single v_bfe_u32.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kChunk = 2048;   // elements per wave chunk (64 lanes x 32)
constexpr int kMaxWaves = 8;

template <int OFF>
__device__ __forceinline__ uint32_t ubfe8(uint32_t v) {
    uint32_t r;
    asm("v_bfe_u32 %0, %1, %2, 8" : "=v"(r) : "v"(v), "i"(OFF));
    return r;
}

struct NF4Smem {
    float lut[16];
    float part[kMaxWaves][16];
};

template <int M, int R>
__global__ __launch_bounds__(kMaxWaves * 64) void nf4_tile_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                                  const uint8_t *__restrict__ codes,
                                                                  const float *__restrict__ absmax, int N, int K,
                                                                  int bs_shift) {
    static_assert(M * R <= 16, "partials buffer");
    __shared__ NF4Smem sm;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    if (threadIdx.x < 16) sm.lut[threadIdx.x] = nf4_level(threadIdx.x);
    __syncthreads();
    const char *lut = reinterpret_cast<const char *>(sm.lut);

    const int row0 = blockIdx.x * R;
    const size_t row_bytes = static_cast<size_t>(K) >> 1;
    const int nchunks = (K + kChunk - 1) / kChunk;

    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int c = wave; c < nchunks; c += S) {
        const int k0 = c * kChunk + lane * 32;
        if (k0 < K) {
            u32x4 q[R];
            float s[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + r, N - 1);
                q[r] = load_stream16(codes + row * row_bytes + (k0 >> 1));
                s[r] = absmax[(static_cast<size_t>(row) * K + k0) >> bs_shift];
            }
            float xv[M][32];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + k0);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 t = xp[i];
                    xv[m][4 * i + 0] = t.x;
                    xv[m][4 * i + 1] = t.y;
                    xv[m][4 * i + 2] = t.z;
                    xv[m][4 * i + 3] = t.w;
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t w[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
                float p[M][2];
#pragma unroll
                for (int m = 0; m < M; ++m) p[m][0] = p[m][1] = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t hi4 = (w[i] >> 2) & 0x3C3C3C3Cu;   // high nibbles * 4 (even elements)
                    const uint32_t lo4 = (w[i] << 2) & 0x3C3C3C3Cu;   // low nibbles * 4 (odd elements)
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
                    for (int m = 0; m < M; ++m)
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            p[m][0] = fmaf(vh[t], xv[m][8 * i + 2 * t], p[m][0]);
                            p[m][1] = fmaf(vl[t], xv[m][8 * i + 2 * t + 1], p[m][1]);
                        }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m][r] = fmaf(p[m][0] + p[m][1], s[r], acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0) sm.part[wave][m * R + r] = v;
        }
    __syncthreads();
    if (threadIdx.x < M * R) {
        const int m = threadIdx.x / R, r = threadIdx.x % R;
        float v = 0.0f;
        for (int w = 0; w < S; ++w) v += sm.part[w][threadIdx.x];
        if (row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
    }
}

// GGUF block codes (see load_gguf_codes in matvec.hip): dwords covering the
// code bytes, realigned with v_alignbit_b32; never reads past the block.
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

struct GgufSmem {
    float part[kMaxWaves][16];
};

// Q4_0 (BYTES=18, NDW=4) and Q8_0 (BYTES=34, NDW=8).
template <int M, int R, bool Q8>
__global__ __launch_bounds__(kMaxWaves * 64) void gguf_tile_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                                   const uint8_t *__restrict__ w, int N, int K) {
    constexpr int NDW = Q8 ? 8 : 4;
    constexpr int BYTES = Q8 ? 34 : 18;
    __shared__ GgufSmem sm;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int S = blockDim.x >> 6;
    const int row0 = blockIdx.x * R;
    const int nblk = K >> 5;
    const size_t row_bytes = static_cast<size_t>(nblk) * BYTES;
    const int nchunks = (nblk + 63) / 64;

    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int c = wave; c < nchunks; c += S) {
        const int b = c * 64 + lane;
        if (b < nblk) {
            uint32_t q[R][NDW];
            float d[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = min(row0 + r, N - 1);
                gguf_block<NDW>(w + row * row_bytes + static_cast<size_t>(b) * BYTES, q[r], d[r]);
            }
            float xv[M][32], xs[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + b * 32);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 t = xp[i];
                    xv[m][4 * i + 0] = t.x;
                    xv[m][4 * i + 1] = t.y;
                    xv[m][4 * i + 2] = t.z;
                    xv[m][4 * i + 3] = t.w;
                }
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    s0 += xv[m][i];
                    s1 += xv[m][16 + i];
                }
                xs[m] = s0 + s1;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float p0 = 0.0f, p1 = 0.0f;
                    if constexpr (!Q8) {
                        // byte j: low nibble -> element j, high nibble -> element 16+j
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t lo = q[r][i] & 0x0F0F0F0Fu;
                            const uint32_t hi = (q[r][i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                p0 = fmaf(static_cast<float>((lo >> (8 * t)) & 0xffu), xv[m][4 * i + t], p0);
                                p1 = fmaf(static_cast<float>((hi >> (8 * t)) & 0xffu), xv[m][16 + 4 * i + t], p1);
                            }
                        }
                        acc[m][r] = fmaf(d[r], fmaf(-8.0f, xs[m], p0 + p1), acc[m][r]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const uint32_t u = q[r][i] ^ 0x80808080u;   // int8 -> biased uint8
#pragma unroll
                            for (int t = 0; t < 4; t += 2) {
                                p0 = fmaf(static_cast<float>((u >> (8 * t)) & 0xffu), xv[m][4 * i + t], p0);
                                p1 = fmaf(static_cast<float>((u >> (8 * t + 8)) & 0xffu), xv[m][4 * i + t + 1], p1);
                            }
                        }
                        acc[m][r] = fmaf(d[r], fmaf(-128.0f, xs[m], p0 + p1), acc[m][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0) sm.part[wave][m * R + r] = v;
        }
    __syncthreads();
    if (threadIdx.x < M * R) {
        const int m = threadIdx.x / R, r = threadIdx.x % R;
        float v = 0.0f;
        for (int ww = 0; ww < S; ++ww) v += sm.part[ww][threadIdx.x];
        if (row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
    }
}

// Rows per workgroup: as many as keep >= ~12 waves per CU busy, up to 8.
int tile_rows(long long N, int S, int cus) {
    for (int R = 8; R > 1; R >>= 1)
        if ((N + R - 1) / R * S >= 12LL * cus) return R;
    return 1;
}

}  // namespace

int enqueue_nf4_tile(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M) {
    if (M > 2 || K % 32 != 0 || bs_shift < 5 || !aligned(Bq, 16) || !aligned(A, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int nchunks = (K + kChunk - 1) / kChunk;
    const int S = nchunks < kMaxWaves ? nchunks : kMaxWaves;
    const int R = tile_rows(N, S, device_cu_count() > 0 ? device_cu_count() : 256);
    const dim3 grid((N + R - 1) / R), block(S * 64);
    hipStream_t s = current_stream();
#define ALJ_NF4_TILE(MM, RR) hipLaunchKernelGGL((nf4_tile_kernel<MM, RR>), grid, block, 0, s, C, A, Bq, absmax, N, K, bs_shift)
    if (M == 1) {
        if (R == 8) ALJ_NF4_TILE(1, 8); else if (R == 4) ALJ_NF4_TILE(1, 4); else if (R == 2) ALJ_NF4_TILE(1, 2); else ALJ_NF4_TILE(1, 1);
    } else {
        if (R == 8) ALJ_NF4_TILE(2, 8); else if (R == 4) ALJ_NF4_TILE(2, 4); else if (R == 2) ALJ_NF4_TILE(2, 2); else ALJ_NF4_TILE(2, 1);
    }
#undef ALJ_NF4_TILE
    return ALJABR_ROCM_OK;
}

int enqueue_gguf_tile(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M) {
    if (M > 2 || (type != ALJABR_ROCM_TYPE_Q4_0 && type != ALJABR_ROCM_TYPE_Q8_0) || K % 32 != 0 ||
        !aligned(A, 16) || !aligned(B, 4))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int nchunks = (K / 32 + 63) / 64;
    const int S = nchunks < kMaxWaves ? nchunks : kMaxWaves;
    const int R = tile_rows(N, S, device_cu_count() > 0 ? device_cu_count() : 256);
    const dim3 grid((N + R - 1) / R), block(S * 64);
    hipStream_t s = current_stream();
#define ALJ_GGUF_TILE(MM, RR, Q8) hipLaunchKernelGGL((gguf_tile_kernel<MM, RR, Q8>), grid, block, 0, s, C, A, B, N, K)
#define ALJ_GGUF_R(MM, Q8)                                  \
    do {                                                    \
        if (R == 8) ALJ_GGUF_TILE(MM, 8, Q8);               \
        else if (R == 4) ALJ_GGUF_TILE(MM, 4, Q8);          \
        else if (R == 2) ALJ_GGUF_TILE(MM, 2, Q8);          \
        else ALJ_GGUF_TILE(MM, 1, Q8);                      \
    } while (0)
    const bool q8 = type == ALJABR_ROCM_TYPE_Q8_0;
    if (M == 1) {
        if (q8) ALJ_GGUF_R(1, true); else ALJ_GGUF_R(1, false);
    } else {
        if (q8) ALJ_GGUF_R(2, true); else ALJ_GGUF_R(2, false);
    }
#undef ALJ_GGUF_R
#undef ALJ_GGUF_TILE
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
