// slice_tails.hip - second kernels of the split-K matrix-core GEMMs that
// consume the K-slice partial sums directly: instead of adding the slices
// into the GEMM outputs and running the decode step's next element-wise
// launch over them, one kernel adds the slices (in slice order, as the plain
// slice sum does) and applies that step:
//   - SwiGLU of the stacked gate/up rows into the FFN activations;
//   - RoPE of the stacked q/k rows, q stored, k and v appended to the fp16
//     caches at each sequence's position;
//   - the residual add of a Wo/down product followed by the next RMSNorm,
//     or, spread over column blocks, the residual add, y * norm_w and the
//     blocks' sums of squares, whose row scale the next GEMM's tail applies.
// Partials are [slice][M][N] over the GEMM's stacked rows N. The arithmetic
// of each step is that of its stand-alone kernel (ops.hip).
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kThreads = 256;

// Sum of one element's slices in slice order, eight loads in flight.
__device__ __forceinline__ float slice_total(const float *__restrict__ part, size_t stride, int slices, size_t idx) {
    return slice_sum(part + idx, stride, slices);
}

__device__ __forceinline__ uint16_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v)); }

// Four consecutive elements (c % 4 == 0) as fp16 (rounded to nearest): one
// 8-byte store.
__device__ __forceinline__ void xpack_store4(uint16_t *xp, int m, int c, int K, float4 v) {
    const uint32_t lo = f16_bits(v.x) | (static_cast<uint32_t>(f16_bits(v.y)) << 16);
    const uint32_t hi = f16_bits(v.z) | (static_cast<uint32_t>(f16_bits(v.w)) << 16);
    *reinterpret_cast<uint2 *>(xp + xpack_index(m, c, K)) = make_uint2(lo, hi);
}

// RMSNorm's row scale 1/sqrt(mean(y^2) + eps) (the sqrt in double, as the
// stand-alone RMSNorm) from the kSsqParts column-block sums of row m, added
// in block order; 1 without sums.
__device__ __forceinline__ float row_scale(const float *ssq, int m, int n, float eps) {
    if (!ssq) return 1.0f;
    float ss = 0.0f;
#pragma unroll
    for (int p = 0; p < kSsqParts; ++p) ss += ssq[m * kSsqParts + p];
    return 1.0f / static_cast<float>(sqrt(static_cast<double>(ss / static_cast<float>(n) + eps)));
}

// GGUFVectorOps.swiGLU (GLD/tensor/GGUFVectorOps.java:333-338): g / (1 + e^-g)
// with the exponential in double, times up.
__device__ __forceinline__ float swiglu_of(float g, float u) {
    return g / (1.0f + static_cast<float>(exp(-static_cast<double>(g)))) * u;
}

// hb[m][i] = swiglu(gate, up) of stacked rows i and n + i (each times the
// row scale of a preceding residual-scale tail, if any).
__global__ __launch_bounds__(kThreads) void tail_swiglu_kernel(float *__restrict__ hb, const float *__restrict__ part,
                                                               int slices, int M, int N, int n,
                                                               const float *__restrict__ ssq, int norm_n, float eps,
                                                               uint16_t *__restrict__ xp) {
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= static_cast<long long>(M) * n) return;
    const int m = static_cast<int>(t / n), i = static_cast<int>(t - static_cast<long long>(m) * n);
    const size_t stride = static_cast<size_t>(M) * N;
    const size_t row = static_cast<size_t>(m) * N;
    const float sc = row_scale(ssq, m, norm_n, eps);
    const float g = slice_total(part, stride, slices, row + i) * sc;
    const float u = slice_total(part, stride, slices, row + n + i) * sc;
    const float h = swiglu_of(g, u);
    hb[t] = h;
    if (xp) xp[xpack_index(m, i, n)] = f16_bits(h);
}

// Workgroup (slot, m), head_dim/2 threads: slots [0, nh) are query heads
// (rotated, stored to q), [nh, nh + nkv) key heads (rotated, appended),
// [nh + nkv, nh + 2 nkv) value heads (appended) - rope_append_kernel's
// arithmetic over the summed partials. Stacked rows: q, then k, then v.
__global__ void tail_rope_append_kernel(float *__restrict__ q, uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                        const int *__restrict__ pos, const float *__restrict__ part, int slices, int M,
                                        int N, int nh, int nkv, int head_dim, int cap, float base,
                                        const float2 *__restrict__ cs, const float *__restrict__ ssq, int norm_n,
                                        float eps) {
    const int slot = blockIdx.x, m = blockIdx.y, i = threadIdx.x;
    const int half = head_dim / 2;
    const size_t stride = static_cast<size_t>(M) * N;
    const size_t row = static_cast<size_t>(m) * N;
    const int p = pos[m];
    float c = 0.0f, s = 0.0f;
    if (slot < nh + nkv) rope_angle(cs, cap, p, i, head_dim, base, c, s);
    // The slot's first stacked row: q heads, then k heads, then v heads,
    // head_dim rows each.
    const size_t r0 = static_cast<size_t>(slot) * head_dim;
    const float sc = row_scale(ssq, m, norm_n, eps);
    float x0 = slice_total(part, stride, slices, row + r0 + i) * sc;
    float x1 = slice_total(part, stride, slices, row + r0 + i + half) * sc;
    if (slot < nh) {
        rope_apply(x0, x1, c, s);
        float *x = q + (static_cast<long long>(m) * nh + slot) * head_dim;
        x[i] = x0;
        x[i + half] = x1;
        return;
    }
    if (p < 0 || p >= cap) return;   // outside the cache: nothing to store
    const int h = slot < nh + nkv ? slot - nh : slot - nh - nkv;
    const long long dst = ((static_cast<long long>(m) * nkv + h) * cap + p) * head_dim;
    if (slot < nh + nkv) {
        rope_apply(x0, x1, c, s);
        kc[dst + i] = f16_bits(x0);
        kc[dst + i + half] = f16_bits(x1);
    } else {
        vc[dst + i] = f16_bits(x0);
        vc[dst + i + half] = f16_bits(x1);
    }
}

__device__ __forceinline__ float tail_block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) t += red[i];
    __syncthreads();
    return t;
}

// One 1024-thread workgroup per row m: y[m] += the summed partials (the
// residual), then xn[m] = RMSNorm(y[m]) * w (1/sqrt in double, (x * scale) *
// w, as the stand-alone RMSNorm). A thread owns float4 columns and keeps
// eight slices' loads in flight (the slices are still added in order).
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void tail_residual_norm_kernel(float *__restrict__ y, float *__restrict__ xn,
                                                                          const float *__restrict__ w, float eps,
                                                                          const float *__restrict__ part, int slices,
                                                                          int M, int N, uint16_t *__restrict__ xp) {
    __shared__ float red[kNormThreads / 64];
    const int m = blockIdx.x;
    const size_t stride = static_cast<size_t>(M) * N;
    const size_t row = static_cast<size_t>(m) * N;
    float4 *yr = reinterpret_cast<float4 *>(y + row);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < N / 4; c += kNormThreads) {
        // The residual row is requested with the partials (one round trip).
        float4 x = yr[c];
        const float4 acc =
            slice_sum(reinterpret_cast<const float4 *>(part + row + 4 * static_cast<size_t>(c)), stride / 4, slices);
        x.x += acc.x;
        x.y += acc.y;
        x.z += acc.z;
        x.w += acc.w;
        yr[c] = x;
        ss = fmaf(x.x, x.x, ss);
        ss = fmaf(x.y, x.y, ss);
        ss = fmaf(x.z, x.z, ss);
        ss = fmaf(x.w, x.w, ss);
    }
    ss = tail_block_sum(ss, red);
    const float scale = 1.0f / static_cast<float>(sqrt(static_cast<double>(ss / static_cast<float>(N) + eps)));
    float4 *xr = reinterpret_cast<float4 *>(xn + row);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    for (int c = threadIdx.x; c < N / 4; c += kNormThreads) {
        const float4 x = yr[c], g = w4[c];
        const float4 o = make_float4((x.x * scale) * g.x, (x.y * scale) * g.y, (x.z * scale) * g.z, (x.w * scale) * g.w);
        xr[c] = o;
        if (xp) xpack_store4(xp, m, 4 * c, N, o);
    }
}

// Workgroup (p, m), 128 threads: column block p (N / kSsqParts columns) of
// row m: y += the summed partials (the residual), xn = y * w, and the block's
// sum of squares of y to ssq[m][p].
constexpr int kScaleThreads = 128;

__global__ __launch_bounds__(kScaleThreads) void tail_residual_scale_kernel(float *__restrict__ y, float *__restrict__ xn,
                                                                            const float *__restrict__ w,
                                                                            float *__restrict__ ssq,
                                                                            const float *__restrict__ part, int slices,
                                                                            int M, int N, uint16_t *__restrict__ xp) {
    __shared__ float red[kScaleThreads / 64];
    const int pb = blockIdx.x, m = blockIdx.y;
    const int cols4 = N / (4 * kSsqParts);              // float4 columns per block
    const size_t stride = static_cast<size_t>(M) * N;
    const size_t row = static_cast<size_t>(m) * N;
    float4 *yr = reinterpret_cast<float4 *>(y + row);
    float4 *xr = reinterpret_cast<float4 *>(xn + row);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float ss = 0.0f;
    for (int c = pb * cols4 + static_cast<int>(threadIdx.x); c < (pb + 1) * cols4; c += kScaleThreads) {
        // The residual row is requested with the partials (one round trip).
        float4 x = yr[c];
        const float4 acc =
            slice_sum(reinterpret_cast<const float4 *>(part + row + 4 * static_cast<size_t>(c)), stride / 4, slices);
        x.x += acc.x;
        x.y += acc.y;
        x.z += acc.z;
        x.w += acc.w;
        yr[c] = x;
        const float4 g = w4[c];
        const float4 o = make_float4(x.x * g.x, x.y * g.y, x.z * g.z, x.w * g.w);
        xr[c] = o;
        if (xp) xpack_store4(xp, m, 4 * c, N, o);
        ss = fmaf(x.x, x.x, ss);
        ss = fmaf(x.y, x.y, ss);
        ss = fmaf(x.z, x.z, ss);
        ss = fmaf(x.w, x.w, ss);
    }
    ss = tail_block_sum(ss, red);
    if (threadIdx.x == 0) ssq[m * kSsqParts + pb] = ss;
}

}  // namespace

int enqueue_slice_tail(const SliceTail &t, const float *part, int slices, int M, int N) {
    hipStream_t s = current_stream();
    switch (t.kind) {
    case kTailSwiGLU: {
        if (2LL * t.n != N || (t.ssq && t.norm_n <= 0) || (t.xpack && (t.n % 64 != 0 || M > 64)))
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        const long long total = static_cast<long long>(M) * t.n;
        hipLaunchKernelGGL(tail_swiglu_kernel, dim3(static_cast<unsigned>((total + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, s, t.out, part, slices, M, N, t.n, t.ssq, t.norm_n, t.eps, t.xpack);
        return ALJABR_ROCM_OK;
    }
    case kTailRopeAppend: {
        if (t.head_dim < 2 || (t.head_dim & 1) || t.head_dim / 2 > 1024 || (t.ssq && t.norm_n <= 0) ||
            static_cast<long long>(t.nh + 2 * t.nkv) * t.head_dim != N)
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(tail_rope_append_kernel, dim3(t.nh + 2 * t.nkv, M), dim3(t.head_dim / 2), 0, s, t.out, t.kc,
                           t.vc, t.pos, part, slices, M, N, t.nh, t.nkv, t.head_dim, t.cap, t.base, t.cs, t.ssq,
                           t.norm_n, t.eps);
        return ALJABR_ROCM_OK;
    }
    case kTailResidualNorm:
        if (N % 4 != 0 || !aligned(t.out, 16) || !aligned(t.xn, 16) || !aligned(t.norm_w, 16) || !aligned(part, 16) ||
            (t.xpack && (N % 64 != 0 || M > 64 || !aligned(t.xpack, 8))))
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(tail_residual_norm_kernel, dim3(M), dim3(kNormThreads), 0, s, t.out, t.xn, t.norm_w, t.eps,
                           part, slices, M, N, t.xpack);
        return ALJABR_ROCM_OK;
    case kTailResidualScale:
        if (N % (4 * kSsqParts) != 0 || !t.ssq || !aligned(t.out, 16) || !aligned(t.xn, 16) ||
            !aligned(t.norm_w, 16) || !aligned(part, 16) || (t.xpack && (N % 64 != 0 || M > 64 || !aligned(t.xpack, 8))))
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        hipLaunchKernelGGL(tail_residual_scale_kernel, dim3(kSsqParts, M), dim3(kScaleThreads), 0, s, t.out, t.xn,
                           t.norm_w, t.ssq, part, slices, M, N, t.xpack);
        return ALJABR_ROCM_OK;
    default: return ALJABR_ROCM_ERR_UNSUPPORTED;
    }
}

}  // namespace aljabr
