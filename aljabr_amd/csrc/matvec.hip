// matvec.hip - batch-1 and small-M (M <= 8) dequant-fused matvec for NF4,
// GGUF Q4_0, GGUF Q8_0 and fp16 rows on gfx950.
//
// Shape: C[m][n] = sum_k A[m][k] * W[n][k], W [N,K] row-major (the
// "transposed right" convention of MTLJ/MetalComputeBackend.java:435-470).
//
// Mapping. One wave64 owns R consecutive rows. The K axis is walked in wave
// chunks: every lane takes one 16-byte slice of packed weights per row per
// chunk (NF4: 32 codes; Q4_0 and Q8_0: one GGUF block), so a chunk is one fully
// coalesced 1 KiB (NF4) / 64-block span per row. Each lane dequantizes in
// registers (NF4 through a 16-entry LDS codebook, conflict-free because at most
// 16 distinct words are read; GGUF codes through v_cvt_f32_ubyte), multiplies
// by the fp32 activations it loaded for its slice (reused across the R rows),
// and keeps per-row partials. One DPP wave reduction per row ends the kernel.
// All arithmetic is fp32 (no packed-fp32 instructions: the build disables them).
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kThreads = 256;   // 4 waves per workgroup

// ---------------------------------------------------------------------------
// NF4: codes u8 [N*K/2] (even element in the high nibble), absmax fp32 over
// the flat element index / blockSize (STC/DequantizationKernel.java:84-102).
// Fast path: K % 32 == 0, blockSize a power of two >= 32.
// ---------------------------------------------------------------------------
template <int M, int R>
__global__ __launch_bounds__(kThreads) void nf4_matvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                              const uint8_t *__restrict__ codes,
                                                              const float *__restrict__ absmax, int N, int K,
                                                              int bs_shift) {
    __shared__ float lut[16];
    if (threadIdx.x < 16) lut[threadIdx.x] = nf4_level(threadIdx.x);
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = ((blockIdx.x * kThreads + threadIdx.x) / kWave) * R;
    if (row0 >= N) return;
    const size_t row_bytes = static_cast<size_t>(K) >> 1;
    const char *lut_bytes = reinterpret_cast<const char *>(lut);

    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int k0 = lane * 32; k0 < K; k0 += kWave * 32) {
        uint4 c[R];
        float s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
            c[r] = *reinterpret_cast<const uint4 *>(codes + row * row_bytes + (k0 >> 1));
            s[r] = absmax[(static_cast<size_t>(row) * K + k0) >> bs_shift];
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float xv[32];
            const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + k0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float4 t = xp[i];
                xv[4 * i + 0] = t.x;
                xv[4 * i + 1] = t.y;
                xv[4 * i + 2] = t.z;
                xv[4 * i + 3] = t.w;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t w[4] = {c[r].x, c[r].y, c[r].z, c[r].w};
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // Byte addresses into the 16-float codebook: nibble * 4.
                    const uint32_t hi4 = (w[i] >> 2) & 0x3C3C3C3Cu;
                    const uint32_t lo4 = (w[i] << 2) & 0x3C3C3C3Cu;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const float vh = *reinterpret_cast<const float *>(lut_bytes + ((hi4 >> (8 * t)) & 0xffu));
                        const float vl = *reinterpret_cast<const float *>(lut_bytes + ((lo4 >> (8 * t)) & 0xffu));
                        p = fmaf(vh, xv[8 * i + 2 * t], p);
                        p = fmaf(vl, xv[8 * i + 2 * t + 1], p);
                    }
                }
                acc[m][r] = fmaf(p, s[r], acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
        }
}

// Any K / even blockSize: one wave per (row, token), lanes stride over bytes.
__global__ __launch_bounds__(kThreads) void nf4_matvec_generic_kernel(float *__restrict__ y,
                                                                      const float *__restrict__ x,
                                                                      const uint8_t *__restrict__ codes,
                                                                      const float *__restrict__ absmax, int N,
                                                                      int K, int M, int bs) {
    const int lane = threadIdx.x & (kWave - 1);
    const int task = (blockIdx.x * kThreads + threadIdx.x) / kWave;
    if (task >= N * M) return;
    const int n = task % N, m = task / N;
    const size_t base = static_cast<size_t>(n) * K;
    const float *xr = x + static_cast<size_t>(m) * K;
    float acc = 0.0f;
    for (int k = lane; k < K; k += kWave) {
        const size_t e = base + k;
        const uint8_t b = codes[e >> 1];
        const int code = (e & 1) ? (b & 15) : (b >> 4);
        acc = fmaf(nf4_level(code) * absmax[e / bs], xr[k], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(m) * N + n] = acc;
}

// ---------------------------------------------------------------------------
// GGUF block loads. A Q4_0 block is 18 bytes ({f16 d; u8 qs[16]}), a Q8_0 block
// 34 bytes; both start at even addresses, so their code bytes start either on
// a dword boundary or 2 bytes past one. Each lane reads the dwords that cover
// its codes and realigns them with v_alignbit_b32; the last two code bytes
// are fetched with a 16-bit load when the block is misaligned, so no read ever
// passes the end of the block.
// ---------------------------------------------------------------------------
template <int NDW>
__device__ __forceinline__ void load_gguf_codes(const uint8_t *blk, uint32_t (&q)[NDW], float &d) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(blk + 2);
    const uint32_t off = static_cast<uint32_t>(a & 3u);   // 0 or 2
    const uint32_t *p = reinterpret_cast<const uint32_t *>(a - off);
    uint32_t dw[NDW + 1];
#pragma unroll
    for (int i = 0; i < NDW; ++i) dw[i] = p[i];
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

// Q4_0: byte j low nibble -> element j, high nibble -> element 16+j
// (GRT/GgufBlockDequantizer.java:403-416). sum (q-8) x = sum q x - 8 sum x.
template <int M, int R>
__global__ __launch_bounds__(kThreads) void q4_0_matvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                               const uint8_t *__restrict__ w, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = ((blockIdx.x * kThreads + threadIdx.x) / kWave) * R;
    if (row0 >= N) return;
    const int nblk = K >> 5;
    const size_t row_bytes = static_cast<size_t>(nblk) * 18;
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int b = lane; b < nblk; b += kWave) {
        uint32_t q[R][4];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
            load_gguf_codes<4>(w + row * row_bytes + static_cast<size_t>(b) * 18, q[r], d[r]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float xv[32];
            const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + b * 32);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float4 t = xp[i];
                xv[4 * i + 0] = t.x;
                xv[4 * i + 1] = t.y;
                xv[4 * i + 2] = t.z;
                xv[4 * i + 3] = t.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) xs += xv[i];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t lo = q[r][i] & 0x0F0F0F0Fu;
                    const uint32_t hi = (q[r][i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        p = fmaf(static_cast<float>((lo >> (8 * t)) & 0xffu), xv[4 * i + t], p);
                        p = fmaf(static_cast<float>((hi >> (8 * t)) & 0xffu), xv[16 + 4 * i + t], p);
                    }
                }
                acc[m][r] = fmaf(d[r], fmaf(-8.0f, xs, p), acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
        }
}

// Q8_0: int8 codes (GRT/GgufBlockDequantizer.java:231-265). Bytes are biased
// to unsigned (xor 0x80) so each converts with one v_cvt_f32_ubyte:
// sum q x = sum (q+128) x - 128 sum x.
template <int M, int R>
__global__ __launch_bounds__(kThreads) void q8_0_matvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                               const uint8_t *__restrict__ w, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = ((blockIdx.x * kThreads + threadIdx.x) / kWave) * R;
    if (row0 >= N) return;
    const int nblk = K >> 5;
    const size_t row_bytes = static_cast<size_t>(nblk) * 34;
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int b = lane; b < nblk; b += kWave) {
        uint32_t q[R][8];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
            load_gguf_codes<8>(w + row * row_bytes + static_cast<size_t>(b) * 34, q[r], d[r]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float xv[32];
            const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + b * 32);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float4 t = xp[i];
                xv[4 * i + 0] = t.x;
                xv[4 * i + 1] = t.y;
                xv[4 * i + 2] = t.z;
                xv[4 * i + 3] = t.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) xs += xv[i];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t u = q[r][i] ^ 0x80808080u;
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        p = fmaf(static_cast<float>((u >> (8 * t)) & 0xffu), xv[4 * i + t], p);
                }
                acc[m][r] = fmaf(d[r], fmaf(-128.0f, xs, p), acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
        }
}

// fp16 rows (LM head, GRT/GgufDenseRows.java:70-90): 8 halves per lane per chunk.
template <int M, int R>
__global__ __launch_bounds__(kThreads) void f16_matvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                              const uint16_t *__restrict__ w, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = ((blockIdx.x * kThreads + threadIdx.x) / kWave) * R;
    if (row0 >= N) return;
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
    for (int k0 = lane * 8; k0 < K; k0 += kWave * 8) {
        uint4 c[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
            c[r] = *reinterpret_cast<const uint4 *>(w + static_cast<size_t>(row) * K + k0);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float4 *xp = reinterpret_cast<const float4 *>(x + static_cast<size_t>(m) * K + k0);
            const float4 xa = xp[0], xb = xp[1];
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t h[4] = {c[r].x, c[r].y, c[r].z, c[r].w};
                float p = acc[m][r];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p = fmaf(f16_bits_to_f32(h[i] & 0xffffu), xv[2 * i], p);
                    p = fmaf(f16_bits_to_f32(h[i] >> 16), xv[2 * i + 1], p);
                }
                acc[m][r] = p;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) y[static_cast<size_t>(m) * N + row0 + r] = v;
        }
}

// fp16 rows with K % 8 != 0 or misaligned rows.
__global__ __launch_bounds__(kThreads) void f16_matvec_generic_kernel(float *__restrict__ y,
                                                                      const float *__restrict__ x,
                                                                      const uint16_t *__restrict__ w, int N, int K,
                                                                      int M) {
    const int lane = threadIdx.x & (kWave - 1);
    const int task = (blockIdx.x * kThreads + threadIdx.x) / kWave;
    if (task >= N * M) return;
    const int n = task % N, m = task / N;
    float acc = 0.0f;
    for (int k = lane; k < K; k += kWave)
        acc = fmaf(f16_bits_to_f32(w[static_cast<size_t>(n) * K + k]), x[static_cast<size_t>(m) * K + k], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(m) * N + n] = acc;
}

// fp32 weight rows (small GGUF models store some matrices unquantized): one
// wave per (row, token), float4 loads when rows allow.
__global__ __launch_bounds__(kThreads) void f32_matvec_kernel(float *__restrict__ y, const float *__restrict__ x,
                                                              const float *__restrict__ w, int N, int K, int M,
                                                              int vec4) {
    const int lane = threadIdx.x & (kWave - 1);
    const int task = (blockIdx.x * kThreads + threadIdx.x) / kWave;
    if (task >= N * M) return;
    const int n = task % N, m = task / N;
    const float *wr = w + static_cast<size_t>(n) * K;
    const float *xr = x + static_cast<size_t>(m) * K;
    float acc = 0.0f;
    if (vec4) {
        for (int k = 4 * lane; k < K; k += 4 * kWave) {
            const float4 a = *reinterpret_cast<const float4 *>(wr + k), b = *reinterpret_cast<const float4 *>(xr + k);
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int k = lane; k < K; k += kWave) acc = fmaf(wr[k], xr[k], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[static_cast<size_t>(m) * N + n] = acc;
}

// ---------------------------------------------------------------------------
// launch helpers
// ---------------------------------------------------------------------------
inline unsigned grid_for(int waves) { return static_cast<unsigned>((waves + 3) / 4); }

// Rows per wave: enough waves to cover every CU several times.
inline int pick_rows(int N) { return N >= 8192 ? 2 : 1; }

template <template <int, int> class>
struct Tag {};

#define ALJ_DISPATCH_MR(KERNEL, M, R, GRID, ...)                                             \
    do {                                                                                     \
        switch ((M) * 8 + (R)) {                                                             \
        case 1 * 8 + 1: hipLaunchKernelGGL((KERNEL<1, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 1 * 8 + 2: hipLaunchKernelGGL((KERNEL<1, 2>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 1 * 8 + 4: hipLaunchKernelGGL((KERNEL<1, 4>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 2 * 8 + 1: hipLaunchKernelGGL((KERNEL<2, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 3 * 8 + 1: hipLaunchKernelGGL((KERNEL<3, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 4 * 8 + 1: hipLaunchKernelGGL((KERNEL<4, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 5 * 8 + 1: hipLaunchKernelGGL((KERNEL<5, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 6 * 8 + 1: hipLaunchKernelGGL((KERNEL<6, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 7 * 8 + 1: hipLaunchKernelGGL((KERNEL<7, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        case 8 * 8 + 1: hipLaunchKernelGGL((KERNEL<8, 1>), GRID, dim3(kThreads), 0, s, __VA_ARGS__); break; \
        default: return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "no %s kernel for M=%d R=%d", #KERNEL, (M), (R)); \
        }                                                                                    \
    } while (0)

}  // namespace

// Small-M GEMMs run on the matrix cores wherever their shape checks pass.
bool mfma_enabled() { return true; }

// Enqueue C[M][N] for M <= 8 (no sync); used by the entry points and the
// decode driver. Returns a status.
int enqueue_nf4_small(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs,
                      int M) {
    hipStream_t s = current_stream();
    const int shift = log2_exact(bs);
    const bool fast = (K % 32 == 0) && shift >= 5 && aligned(Bq, 16) && aligned(A, 16);
    if (!fast) {
        hipLaunchKernelGGL(nf4_matvec_generic_kernel, dim3(grid_for(N * M)), dim3(kThreads), 0, s, C, A, Bq, absmax,
                           N, K, M, bs);
        return ALJABR_ROCM_OK;
    }
    // Batch 1: the rows kernel (K % 2048 == 0, at most 8 chunks), else the
    // per-workgroup rows kernel (up to 16 chunks), else the tile kernel.
    if (M == 1 && enqueue_rows(C, A, Bq, absmax, K, N, ALJABR_ROCM_TYPE_NF4, shift) == ALJABR_ROCM_OK)
        return ALJABR_ROCM_OK;
    if (M == 1 && enqueue_nf4_rows(C, A, Bq, absmax, K, N, shift) == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
    if (enqueue_nf4_tile(C, A, Bq, absmax, K, N, shift, M) == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
    const int R = M == 1 ? pick_rows(N) : 1;
    const dim3 grid(grid_for((N + R - 1) / R));
    ALJ_DISPATCH_MR(nf4_matvec_kernel, M, R, grid, C, A, Bq, absmax, N, K, shift);
    return ALJABR_ROCM_OK;
}

int enqueue_gguf_small(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M) {
    hipStream_t s = current_stream();
    if (type != ALJABR_ROCM_TYPE_F16 && (!aligned(A, 16) || !aligned(B, 4)))
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "GGUF matvec needs A 16-byte and B 4-byte aligned");
    if (M == 1 && type != ALJABR_ROCM_TYPE_F16 &&
        enqueue_rows(C, A, B, nullptr, K, N, type, 0) == ALJABR_ROCM_OK)
        return ALJABR_ROCM_OK;
    if (M == 1 && enqueue_gguf_stream(C, A, B, K, N, type) == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
    if (enqueue_gguf_tile(C, A, B, K, N, type, M) == ALJABR_ROCM_OK) return ALJABR_ROCM_OK;
    const int R = M == 1 ? pick_rows(N) : 1;
    const dim3 grid(grid_for((N + R - 1) / R));
    if (type == ALJABR_ROCM_TYPE_Q4_0) {
        ALJ_DISPATCH_MR(q4_0_matvec_kernel, M, R, grid, C, A, B, N, K);
    } else if (type == ALJABR_ROCM_TYPE_Q8_0) {
        ALJ_DISPATCH_MR(q8_0_matvec_kernel, M, R, grid, C, A, B, N, K);
    } else {
        const uint16_t *W = reinterpret_cast<const uint16_t *>(B);
        if (K % 8 == 0 && aligned(B, 16) && aligned(A, 16)) {
            ALJ_DISPATCH_MR(f16_matvec_kernel, M, R, grid, C, A, W, N, K);
        } else {
            hipLaunchKernelGGL(f16_matvec_generic_kernel, dim3(grid_for(N * M)), dim3(kThreads), 0, s, C, A, W, N, K,
                               M);
        }
    }
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr

using namespace aljabr;

namespace aljabr {

// M > 8 slices run the small-M kernels per slice of 8 tokens (weights are
// re-read per slice); the MFMA path takes over at its threshold.
int enqueue_matmul_nf4(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs, int M,
                       float *part, size_t part_floats) {
    // M = 2..4 on the batch-1 rows kernel (fp32, the weights streamed once).
    if (M >= 2 && M <= 4) {
        const int shift = log2_exact(bs);
        if (shift >= 0 && enqueue_rows_nf4_mt(C, A, Bq, absmax, K, N, shift, M) == ALJABR_ROCM_OK)
            return ALJABR_ROCM_OK;
    }
    // M >= 2 on the matrix cores when the shape allows (deterministic;
    // passes of 64 tokens).
    if (M >= 2 && mfma_enabled()) {
        const int shift = log2_exact(bs);
        const int rc = enqueue_nf4_mfma(C, A, Bq, absmax, K, N, shift, M, false, part, part_floats);
        if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
    }
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mm = M - m0 < 8 ? M - m0 : 8;
        int rc = enqueue_nf4_small(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, Bq, absmax, K, N,
                                   bs, mm);
        if (rc != ALJABR_ROCM_OK) return rc;
    }
    return ALJABR_ROCM_OK;
}

int enqueue_matmul_gguf(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M, float *part,
                        size_t part_floats) {
    if (type == ALJABR_ROCM_TYPE_Q4_K || type == ALJABR_ROCM_TYPE_Q6_K)
        return enqueue_matmul_kquant(C, A, B, K, N, type, M, part, part_floats);
    // Q4_0 / Q8_0 with M >= 2 on the matrix cores (K % 512, 16-byte aligned),
    // 8 tokens per pass; a last single token takes the batch-1 path.
    if ((type == ALJABR_ROCM_TYPE_Q4_0 || type == ALJABR_ROCM_TYPE_Q8_0) && M >= 2 && K % 512 == 0 &&
        aligned(A, 16) && aligned(B, 16) && mfma_enabled()) {
        int m0 = 0;
        while (M - m0 >= 2) {
            const int mm = M - m0 < 8 ? M - m0 : 8;
            const int rc = enqueue_kquant_mfma(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, B, K,
                                               N, type, mm, part, part_floats);
            if (rc != ALJABR_ROCM_OK) return rc;
            m0 += mm;                            // the pass covered exactly mm tokens
        }
        if (m0 == M) return ALJABR_ROCM_OK;      // otherwise exactly one token is left
        return enqueue_gguf_small(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, B, K, N, type, 1);
    }
    // fp16 rows with M >= 2 on the matrix cores, 32 tokens per pass.
    if (type == ALJABR_ROCM_TYPE_F16 && M >= 2 && mfma_enabled()) {
        const uint16_t *W = reinterpret_cast<const uint16_t *>(B);
        bool ok = true;
        for (int m0 = 0; m0 < M && ok; m0 += 32) {
            const int mm = M - m0 < 32 ? M - m0 : 32;
            int rc;
            if (mm >= 2) {
                rc = enqueue_f16_mfma(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, W, K, N, mm);
                if (rc == ALJABR_ROCM_ERR_UNSUPPORTED && m0 == 0) {   // the shape checks do not depend on m0
                    ok = false;
                    break;
                }
            } else {
                rc = enqueue_gguf_small(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, B, K, N,
                                        type, 1);
            }
            if (rc != ALJABR_ROCM_OK) return rc;
        }
        if (ok) return ALJABR_ROCM_OK;
    }
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mm = M - m0 < 8 ? M - m0 : 8;
        int rc = enqueue_gguf_small(C + static_cast<size_t>(m0) * N, A + static_cast<size_t>(m0) * K, B, K, N, type,
                                    mm);
        if (rc != ALJABR_ROCM_OK) return rc;
    }
    return ALJABR_ROCM_OK;
}

int enqueue_matmul_f32(float *C, const float *A, const float *W, int K, int N, int M) {
    const long long tasks = static_cast<long long>(N) * M;
    if (tasks > 0x7fffffffLL / 64) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int vec4 = K % 4 == 0 && aligned(A, 16) && aligned(W, 16);
    hipLaunchKernelGGL(f32_matvec_kernel, dim3(grid_for(static_cast<int>(tasks))), dim3(kThreads), 0,
                       current_stream(), C, A, W, N, K, M, vec4);
    return ALJABR_ROCM_OK;
}

int enqueue_matmul_typed(float *C, const float *A, const void *W, const float *absmax, int type, int bs, int K, int N,
                         int M, float *part, size_t part_floats) {
    const uint8_t *w = static_cast<const uint8_t *>(W);
    switch (type) {
    case ALJABR_ROCM_TYPE_NF4: return enqueue_matmul_nf4(C, A, w, absmax, K, N, bs, M, part, part_floats);
    case ALJABR_ROCM_TYPE_F32: return enqueue_matmul_f32(C, A, static_cast<const float *>(W), K, N, M);
    case ALJABR_ROCM_TYPE_F16:
    case ALJABR_ROCM_TYPE_Q4_0:
    case ALJABR_ROCM_TYPE_Q8_0:
    case ALJABR_ROCM_TYPE_Q4_K:
    case ALJABR_ROCM_TYPE_Q6_K: return enqueue_matmul_gguf(C, A, w, K, N, type, M, part, part_floats);
    default: return ALJABR_ROCM_ERR_UNSUPPORTED;
    }
}

}  // namespace aljabr

namespace {

int check_common(const void *C, const void *A, const void *B, int K, int N, int batch) {
    ALJ_REQUIRE(C && A && B, "C, A and B must be non-null device pointers");
    ALJ_REQUIRE(K > 0 && N > 0 && batch > 0, "bad dimensions K=%d N=%d batch=%d", K, N, batch);
    return ALJABR_ROCM_OK;
}

}  // namespace

extern "C" {

int aljabr_rocm_matvec_tb_batch_nf4(void *C, const void *A, const void *B_packed, const void *absmax, int K, int N,
                                    int blockSize, int batchSize) {
    ALJ_CHECK_READY();
    int rc = check_common(C, A, B_packed, K, N, batchSize);
    if (rc) return rc;
    ALJ_REQUIRE(absmax, "absmax must be a non-null device pointer");
    ALJ_REQUIRE(blockSize > 0 && blockSize % 2 == 0, "NF4 blockSize must be positive and even (got %d)", blockSize);
    rc = enqueue_matmul_nf4(static_cast<float *>(C), static_cast<const float *>(A), static_cast<const uint8_t *>(B_packed),
                 static_cast<const float *>(absmax), K, N, blockSize, batchSize);
    if (rc) return rc;
    return finish_launch("matvec_tb_batch_nf4");
}

int aljabr_rocm_matvec_tb_nf4(void *C, const void *A, const void *B_packed, const void *absmax, int K, int N,
                              int blockSize) {
    return aljabr_rocm_matvec_tb_batch_nf4(C, A, B_packed, absmax, K, N, blockSize, 1);
}

int aljabr_rocm_matvec_tb_batch(void *C, const void *A, const void *B, int K, int N, int type, int batchSize) {
    ALJ_CHECK_READY();
    int rc = check_common(C, A, B, K, N, batchSize);
    if (rc) return rc;
    const bool kq = type == ALJABR_ROCM_TYPE_Q4_K || type == ALJABR_ROCM_TYPE_Q6_K;
    if (type != ALJABR_ROCM_TYPE_Q4_0 && type != ALJABR_ROCM_TYPE_Q8_0 && type != ALJABR_ROCM_TYPE_F16 && !kq)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "matvec_tb_batch: unsupported type %d", type);
    if (kq) ALJ_REQUIRE(K % 256 == 0, "K-quant rows are whole 256-element super-blocks (K=%d)", K);
    else if (type != ALJABR_ROCM_TYPE_F16) ALJ_REQUIRE(K % 32 == 0, "GGUF rows are whole 32-element blocks (K=%d)", K);
    rc = enqueue_matmul_gguf(static_cast<float *>(C), static_cast<const float *>(A), static_cast<const uint8_t *>(B), K, N, type,
                  batchSize);
    if (rc) return rc;
    return finish_launch("matvec_tb_batch");
}

int aljabr_rocm_matvec_tb_q4_0(void *C, const void *A, const void *B, int K, int N) {
    return aljabr_rocm_matvec_tb_batch(C, A, B, K, N, ALJABR_ROCM_TYPE_Q4_0, 1);
}

int aljabr_rocm_matvec_tb_q8_0(void *C, const void *A, const void *B, int K, int N) {
    return aljabr_rocm_matvec_tb_batch(C, A, B, K, N, ALJABR_ROCM_TYPE_Q8_0, 1);
}

int aljabr_rocm_matvec_tb_half(void *C, const void *A, const void *B, int K, int N) {
    return aljabr_rocm_matvec_tb_batch(C, A, B, K, N, ALJABR_ROCM_TYPE_F16, 1);
}

int aljabr_rocm_matvec_tb_q4_k(void *C, const void *A, const void *B, int K, int N) {
    return aljabr_rocm_matvec_tb_batch(C, A, B, K, N, ALJABR_ROCM_TYPE_Q4_K, 1);
}

int aljabr_rocm_matvec_tb_q6_k(void *C, const void *A, const void *B, int K, int N) {
    return aljabr_rocm_matvec_tb_batch(C, A, B, K, N, ALJABR_ROCM_TYPE_Q6_K, 1);
}

}  // extern "C"

namespace {

// The soft-capped variants run the matvec and then the cap in the same stream
// (as Metal's fallback path does when it has no fused pipeline).
int matvec_softcap(void *C, const void *A, const void *B, int K, int N, int type, float cap) {
    ALJ_CHECK_READY();
    int rc = check_common(C, A, B, K, N, 1);
    if (rc) return rc;
    ALJ_REQUIRE(K % 256 == 0, "K-quant rows are whole 256-element super-blocks (K=%d)", K);
    ALJ_REQUIRE(!(cap != cap), "cap must not be NaN");
    rc = enqueue_matmul_kquant(static_cast<float *>(C), static_cast<const float *>(A), static_cast<const uint8_t *>(B),
                               K, N, type, 1);
    if (rc) return rc;
    if (cap > 0.0f) enqueue_softcap(static_cast<float *>(C), N, cap);
    return finish_launch("matvec_tb_softcap");
}

}  // namespace

extern "C" {

int aljabr_rocm_matvec_tb_q4_k_softcap(void *C, const void *A, const void *B, int K, int N, float cap) {
    return matvec_softcap(C, A, B, K, N, ALJABR_ROCM_TYPE_Q4_K, cap);
}

int aljabr_rocm_matvec_tb_q6_k_softcap(void *C, const void *A, const void *B, int K, int N, float cap) {
    return matvec_softcap(C, A, B, K, N, ALJABR_ROCM_TYPE_Q6_K, cap);
}

}  // extern "C"
