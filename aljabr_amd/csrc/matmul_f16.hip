// matmul_f16.hip - fp16-weight small-M GEMM on the matrix cores:
// Y[M,N] = X[M,K] . W[N,K]^T with W in IEEE half (the decode step's LM head,
// GGUF F16 rows: GRT/GgufDenseRows.java:70-90) and 2 <= M <= 32 per pass.
// Replaces one pass over W per token (or per slice of 8 tokens) with one pass
// for the whole batch: at M = 32 the 1 GB LM head is read once instead of 4
// times.
//
// MFMA v_mfma_f32_32x32x16_f16, A = X rounded to fp16 (relative error
// <= 2^-11 per element), B = W^T as stored, fp32 accumulation.
//
// Work split: a workgroup is 8 waves; wave w owns the K-slice
// [w*K/8, (w+1)*K/8) and keeps that slice of X for all 32 token rows in
// registers as MFMA A fragments (K/32 VGPRs), loaded once. The workgroup walks
// 32-row tiles of W (tile = blockIdx.x + i*gridDim.x); per tile each wave
// contracts its slice and the 8 partial tiles are summed through LDS, so no
// atomics and no clearing pass are needed and results are deterministic.
//
// Operand layout (32x32x16): lane l supplies A[m = l%32][8*(l/32) + e] and
// B[8*(l/32) + e][n = l%32]; accumulator r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32]. The contraction index is permuted so a
// 64-element step of K is four MFMAs: lane half h supplies k = 32h + 8j + e
// for MFMA j of the step (A and B use the same map).
//
// Loads are coalesced (8 lanes read one row's 128-byte step segment; the MFMA
// layout would touch 32 lines per instruction) and transposed through a
// per-wave LDS staging block with a 144-byte row stride (conflict-free both
// ways). Loads run D steps ahead of the step being computed, across tile
// boundaries.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kStageStride = 144;                // bytes per staged row: 128 + 16 pad

struct F16MmArgs {
    float *y;
    const float *x;
    const uint16_t *w;
    int M, N, K;
};

// Coalesced loads of step s of tile t: instruction i covers rows
// 8i + lane/8 of the tile, elements 8*(lane%8) of the row's 64-element step.
__device__ __forceinline__ void issue_step(u32x4 (&q)[4], const F16MmArgs &a, int tile, int k0, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = min(tile * 32 + 8 * i + (lane >> 3), a.N - 1);
        q[i] = load_stream16(a.w + static_cast<size_t>(row) * a.K + k0 + 8 * (lane & 7));
    }
}

__device__ __forceinline__ half8 to_half8(f32x4 lo, f32x4 hi) {
    half8 r;
    r[0] = static_cast<_Float16>(lo.x); r[1] = static_cast<_Float16>(lo.y);
    r[2] = static_cast<_Float16>(lo.z); r[3] = static_cast<_Float16>(lo.w);
    r[4] = static_cast<_Float16>(hi.x); r[5] = static_cast<_Float16>(hi.y);
    r[6] = static_cast<_Float16>(hi.z); r[7] = static_cast<_Float16>(hi.w);
    return r;
}

template <int KSTEPS, int D>
__global__ __launch_bounds__(kThreads) void f16_mm_kernel(F16MmArgs a) {
    static_assert(KSTEPS % D == 0, "load ring must divide the steps of a tile");
    __shared__ float red[2][kWaves][16][64];
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][32 * kStageStride];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 31, h = lane >> 5;
    const int kw0 = wave * (KSTEPS * 64);
    const int ntiles = (a.N + 31) >> 5;
    int tile = blockIdx.x;                       // the grid never exceeds the tile count

    // This wave's K-slice of X as A fragments, rows >= M zero.
    half8 af[KSTEPS][4];
    {
        const bool mv = nl < a.M;
        const float *xr = a.x + static_cast<size_t>(mv ? nl : 0) * a.K + kw0 + 32 * h;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 lo = *reinterpret_cast<const f32x4 *>(xr + 64 * s + 8 * j);
                f32x4 hi = *reinterpret_cast<const f32x4 *>(xr + 64 * s + 8 * j + 4);
                if (!mv) lo = hi = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                af[s][j] = to_half8(lo, hi);
            }
    }
    __builtin_amdgcn_sched_barrier(0);           // activations before the weight stream

    u32x4 ring[D][4];
#pragma unroll
    for (int s = 0; s < D; ++s) issue_step(ring[s], a, tile, kw0 + 64 * s, lane);

    uint8_t *st = stage[wave];
    int buf = 0;
    for (;;) {
        const int next = tile + gridDim.x;
        const bool more = next < ntiles;
        f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            u32x4 cur[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = ring[s % D][i];
            // Branch-free refill (the last tile re-reads its own first steps):
            // a conditional load here makes the compiler drain every load in
            // flight at the join.
            if (s + D < KSTEPS) issue_step(ring[s % D], a, tile, kw0 + 64 * (s + D), lane);
            else issue_step(ring[s % D], a, more ? next : tile, kw0 + 64 * (s + D - KSTEPS), lane);
            // Rows to the MFMA layout (a wave's LDS operations run in order,
            // so the next step's writes never overtake these reads).
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<u32x4 *>(st + (8 * i + (lane >> 3)) * kStageStride + 16 * (lane & 7)) = cur[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8 bf = *reinterpret_cast<const half8 *>(st + nl * kStageStride + 64 * h + 16 * j);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s][j], bf, acc, 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Sum the 8 K-slices of the tile: thread (g = tid/64, l2 = tid%64)
        // takes accumulators 2g and 2g+1 of lane l2.
#pragma unroll
        for (int r = 0; r < 16; ++r) red[buf][wave][r][lane] = acc[r];
        lds_barrier();
        {
            const int g = tid >> 6, l2 = tid & 63;
            const int n = tile * 32 + (l2 & 31);
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int r = 2 * g + rr;
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) v += red[buf][w][r][l2];
                const int m = 8 * (r >> 2) + 4 * (l2 >> 5) + (r & 3);
                if (m < a.M && n < a.N) a.y[static_cast<size_t>(m) * a.N + n] = v;
            }
        }
        buf ^= 1;
        if (!more) break;
        tile = next;
    }
}

template <int KSTEPS, int D>
void launch_f16(const F16MmArgs &args, hipStream_t s) {
    const int ntiles = (args.N + 31) / 32;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int grid = ntiles < cus ? ntiles : cus;
    hipLaunchKernelGGL((f16_mm_kernel<KSTEPS, D>), dim3(grid), dim3(kThreads), 0, s, args);
}

}  // namespace

// 2 <= M <= 32, K in {512, 1024, 2048, 4096}, W rows and X 16-byte aligned.
int enqueue_f16_mfma(float *C, const float *A, const uint16_t *W, int K, int N, int M) {
    if (M < 2 || M > 32 || N < 1 || !aligned(A, 16) || !aligned(W, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const F16MmArgs args{C, A, W, M, N, K};
    hipStream_t s = current_stream();
    switch (K) {
    case 512: launch_f16<1, 1>(args, s); break;
    case 1024: launch_f16<2, 2>(args, s); break;
    case 2048: launch_f16<4, 4>(args, s); break;
    case 4096: launch_f16<8, 2>(args, s); break;
    default: return ALJABR_ROCM_ERR_UNSUPPORTED;
    }
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr
