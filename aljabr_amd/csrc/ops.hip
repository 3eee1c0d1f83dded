// ops.hip - decode-step element-wise kernels (fp32): RMSNorm, split-half RoPE,
// SwiGLU, residual add, argmax, token-embedding gather and fp16 KV append.
//
// Arithmetic follows GLD/tensor/GGUFVectorOps.java (engine/gguf/aljabr-gguf-core/
// src/main/java/tech/kayys/aljabr/gguf/loader/tensor): rmsNorm :211-234,
// swiGLU :333-338, rope :383-440, addInPlace :108-116. Transcendentals that
// the reference evaluates in double (Math.sqrt/exp/pow/cos/sin) are evaluated
// in double here too.
#include <cmath>

#include "dequant.hpp"
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) t += red[i];
    __syncthreads();
    return t;
}

// One workgroup per row. With len % 4 == 0 and 16-byte aligned rows every
// thread issues its float4 loads back to back (four in flight) instead of one
// dependent scalar load per trip.
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(float *__restrict__ out, const float *__restrict__ x,
                                                           const float *__restrict__ w, int rows, int len, float eps) {
    if (static_cast<int>(blockIdx.x) >= rows) return;
    __shared__ float red[kThreads / 64];
    const float *xr = x + static_cast<long long>(blockIdx.x) * len;
    float *orow = out + static_cast<long long>(blockIdx.x) * len;
    const bool vec = (len & 3) == 0 && ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(orow) |
                                         reinterpret_cast<uintptr_t>(w)) & 15) == 0;
    const int n4 = len >> 2;
    float ss = 0.0f;
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        for (int base = threadIdx.x; base < n4; base += 4 * kThreads) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = base + u * kThreads;
                v[u] = i < n4 ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ss = fmaf(v[u].x, v[u].x, ss);
                ss = fmaf(v[u].y, v[u].y, ss);
                ss = fmaf(v[u].z, v[u].z, ss);
                ss = fmaf(v[u].w, v[u].w, ss);
            }
        }
    } else {
        for (int i = threadIdx.x; i < len; i += kThreads) ss = fmaf(xr[i], xr[i], ss);
    }
    ss = block_sum(ss, red);
    const float scale = 1.0f / static_cast<float>(sqrt(static_cast<double>(ss / static_cast<float>(len) + eps)));
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        const float4 *w4 = reinterpret_cast<const float4 *>(w);
        float4 *o4 = reinterpret_cast<float4 *>(orow);
        for (int base = threadIdx.x; base < n4; base += 4 * kThreads) {
            float4 v[4], g[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = base + u * kThreads;
                if (i < n4) {
                    v[u] = x4[i];
                    g[u] = w4[i];
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = base + u * kThreads;
                if (i < n4)
                    o4[i] = make_float4((v[u].x * scale) * g[u].x, (v[u].y * scale) * g[u].y,
                                        (v[u].z * scale) * g[u].z, (v[u].w * scale) * g[u].w);
            }
        }
    } else {
        for (int i = threadIdx.x; i < len; i += kThreads) orow[i] = (xr[i] * scale) * w[i];
    }
}

// Split-half rotation of the pair (i, i + D/2) at position `pos`
// (GGUFVectorOps.rope :383-440): invFreq = base^(-2i/D) and cos/sin in double.
__device__ __forceinline__ void rope_pair(float &x0, float &x1, int pos, int i, int head_dim, float base) {
    float c, s;
    rope_cos_sin(pos, i, head_dim, base, c, s);
    rope_apply(x0, x1, c, s);
}

// One thread per (position, pair): the decode step's cos/sin table.
__global__ __launch_bounds__(kThreads) void rope_table_kernel(float2 *__restrict__ cs, int cap, int head_dim,
                                                              float base) {
    const int half = head_dim / 2;
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (t >= static_cast<long long>(cap) * half) return;
    float c, s;
    rope_cos_sin(static_cast<int>(t / half), static_cast<int>(t % half), head_dim, base, c, s);
    cs[t] = make_float2(c, s);
}

// One thread per (row, head, pair i < half).
__global__ __launch_bounds__(kThreads) void rope_kernel(float *__restrict__ x, const int *__restrict__ pos, int rows,
                                                        int n_heads, int head_dim, float base) {
    const int half = head_dim / 2;
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    const long long total = static_cast<long long>(rows) * n_heads * half;
    if (t >= total) return;
    const int i = static_cast<int>(t % half);
    const long long rh = t / half;   // row * n_heads + head
    const int row = static_cast<int>(rh / n_heads);
    float *p = x + rh * head_dim;
    float x0 = p[i], x1 = p[i + half];
    rope_pair(x0, x1, pos[row], i, head_dim, base);
    p[i] = x0;
    p[i + half] = x1;
}

__device__ __forceinline__ uint16_t to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// The decode step's RoPE + KV append in one launch: workgroup (slot, b) with
// D/2 threads; slots [0, nh) rotate query heads in place, [nh, nh + nkv)
// rotate key heads and store them as fp16 at cache row pos[b], and
// [nh + nkv, nh + 2 nkv) store value heads. Same arithmetic as rope_kernel
// followed by kv_append_kernel.
__global__ void rope_append_kernel(float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
                                   uint16_t *__restrict__ kc, uint16_t *__restrict__ vc, const int *__restrict__ pos,
                                   int nh, int nkv, int head_dim, int cap, float base, const float2 *__restrict__ cs) {
    const int slot = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int half = head_dim / 2;
    const int p = pos[b];
    float c = 0.0f, s = 0.0f;
    if (slot < nh + nkv) rope_angle(cs, cap, p, i, head_dim, base, c, s);
    if (slot < nh) {
        float *x = q + (static_cast<long long>(b) * nh + slot) * head_dim;
        float x0 = x[i], x1 = x[i + half];
        rope_apply(x0, x1, c, s);
        x[i] = x0;
        x[i + half] = x1;
        return;
    }
    if (p < 0 || p >= cap) return;   // outside the cache: nothing to store
    const int h = slot < nh + nkv ? slot - nh : slot - nh - nkv;
    const long long src = (static_cast<long long>(b) * nkv + h) * head_dim;
    const long long dst = ((static_cast<long long>(b) * nkv + h) * cap + p) * head_dim;
    if (slot < nh + nkv) {
        float x0 = k[src + i], x1 = k[src + i + half];
        rope_apply(x0, x1, c, s);
        kc[dst + i] = to_f16_bits(x0);
        kc[dst + i + half] = to_f16_bits(x1);
    } else {
        vc[dst + i] = to_f16_bits(v[src + i]);
        vc[dst + i + half] = to_f16_bits(v[src + i + half]);
    }
}

__device__ __forceinline__ float swiglu_one(float g, float u) {
    const float sg = g / (1.0f + static_cast<float>(exp(-static_cast<double>(g))));
    return sg * u;
}

// Four elements per thread (float4) when all three arrays are 16-byte aligned.
__global__ __launch_bounds__(kThreads) void swiglu_kernel(float *__restrict__ dst, const float *__restrict__ gate,
                                                          const float *__restrict__ up, long long n) {
    const long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(gate) |
                       reinterpret_cast<uintptr_t>(up)) & 15) == 0;
    if (vec) {
        const long long i = 4 * t;
        if (i + 3 < n) {
            const float4 g = *reinterpret_cast<const float4 *>(gate + i);
            const float4 u = *reinterpret_cast<const float4 *>(up + i);
            *reinterpret_cast<float4 *>(dst + i) =
                make_float4(swiglu_one(g.x, u.x), swiglu_one(g.y, u.y), swiglu_one(g.z, u.z), swiglu_one(g.w, u.w));
        } else {
            for (long long j = i; j < n; ++j) dst[j] = swiglu_one(gate[j], up[j]);
        }
    } else {
        for (long long j = 4 * t; j < 4 * t + 4 && j < n; ++j) dst[j] = swiglu_one(gate[j], up[j]);
    }
}

__global__ __launch_bounds__(kThreads) void add_kernel(float *__restrict__ a, const float *__restrict__ b, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) a[i] += b[i];
}

__device__ __forceinline__ void argmax_take(float v, int i, float &best, int &bi) {
    if (v > best || (v == best && i < bi)) {
        best = v;
        bi = i;
    }
}

// Wide rows in two launches: workgroup (c, r) finds the maximum of chunk c
// (kArgmaxChunk columns) of row r with the lowest index among equal values
// and stores it; one wave per row then takes the best of its chunks' results
// by the same rule. NaN is never taken, and a row with nothing above -inf
// yields 0, as in argmax_kernel. The result does not depend on the order in
// which candidates meet (value first, then the lower index).
constexpr int kArgmaxChunk = 2048;
constexpr int kArgmaxThreads = 256;
struct ArgmaxPart {
    float v;
    int i;
};

__device__ __forceinline__ void argmax_wave(float &best, int &bi) {
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(bi, off);
        argmax_take(ov, oi, best, bi);
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_chunk_kernel(ArgmaxPart *__restrict__ part,
                                                                      const float *__restrict__ x, int cols) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const float *row = x + static_cast<long long>(blockIdx.y) * cols;
    const int c0 = blockIdx.x * kArgmaxChunk;
    const int c1 = min(c0 + kArgmaxChunk, cols);
    float best = -INFINITY;
    int bi = 0x7fffffff;
    if ((cols & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        // float4 j of the chunk: columns c0 + 4j .. +3 (c1 - c0 is a multiple of 4).
        const float4 *r4 = reinterpret_cast<const float4 *>(row + c0);
        const int n4 = (c1 - c0) >> 2;
        float4 v[kArgmaxChunk / 4 / kArgmaxThreads];
#pragma unroll
        for (int u = 0; u < kArgmaxChunk / 4 / kArgmaxThreads; ++u) {
            const int j = threadIdx.x + u * kArgmaxThreads;
            v[u] = j < n4 ? r4[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int u = 0; u < kArgmaxChunk / 4 / kArgmaxThreads; ++u) {
            const int i = c0 + 4 * (threadIdx.x + u * kArgmaxThreads);
            argmax_take(v[u].x, i, best, bi);
            argmax_take(v[u].y, i + 1, best, bi);
            argmax_take(v[u].z, i + 2, best, bi);
            argmax_take(v[u].w, i + 3, best, bi);
        }
    } else {
        for (int i = c0 + static_cast<int>(threadIdx.x); i < c1; i += kArgmaxThreads) argmax_take(row[i], i, best, bi);
    }
    argmax_wave(best, bi);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kArgmaxThreads / 64; ++k) argmax_take(sv[k], si[k], best, bi);
        part[static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x] = ArgmaxPart{best, bi};
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(int *__restrict__ out, const ArgmaxPart *__restrict__ part,
                                                          int chunks) {
    const ArgmaxPart *pr = part + static_cast<size_t>(blockIdx.x) * chunks;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int c = threadIdx.x; c < chunks; c += 64) argmax_take(pr[c].v, pr[c].i, best, bi);
    argmax_wave(best, bi);
    if (threadIdx.x == 0) out[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
}

// One 1024-thread workgroup per row; ties resolve to the lowest index. Rows
// of 16-byte aligned float4s are read eight loads per thread per trip.
__global__ __launch_bounds__(1024) void argmax_kernel(int *__restrict__ out, const float *__restrict__ x, int cols) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const float *row = x + static_cast<long long>(blockIdx.x) * cols;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    if ((cols & 3) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = cols >> 2;
        for (int base = threadIdx.x; base < n4; base += 8 * 1024) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = base + u * 1024;
                v[u] = i < n4 ? r4[i] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (base + u * 1024 >= n4) break;
                const int i = 4 * (base + u * 1024);
                argmax_take(v[u].x, i, best, bi);
                argmax_take(v[u].y, i + 1, best, bi);
                argmax_take(v[u].z, i + 2, best, bi);
                argmax_take(v[u].w, i + 3, best, bi);
            }
        }
    } else {
        for (int i = threadIdx.x; i < cols; i += 1024) argmax_take(row[i], i, best, bi);
    }
    // Wave reduction with index tie-break.
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(bi, off);
        argmax_take(ov, oi, best, bi);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 16; ++k) argmax_take(sv[k], si[k], best, bi);
        out[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
    }
}

// x[b][:] = embed[tokens[b]][:]
__global__ __launch_bounds__(kThreads) void embed_kernel(float *__restrict__ x, const float *__restrict__ embed,
                                                         const int *__restrict__ tokens, int dim, int vocab) {
    const int b = blockIdx.y;
    int t = tokens[b];
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < dim; i += gridDim.x * kThreads)
        x[static_cast<long long>(b) * dim + i] = embed[static_cast<long long>(t) * dim + i];
}

// One thread per 32 elements of row tokens[b]: a Q4_0 / Q8_0 block, a Q4_K
// sub-block, two Q6_K scale groups, or 32 fp16 / fp32 values.
__global__ __launch_bounds__(kThreads) void embed_typed_kernel(float *__restrict__ x, const uint8_t *__restrict__ table,
                                                               int type, const int *__restrict__ tokens, int dim,
                                                               int vocab, long long row_bytes) {
    const int b = blockIdx.y;
    const int u = blockIdx.x * kThreads + threadIdx.x;      // 32-element unit of the row
    if (32 * u >= dim) return;
    int t = tokens[b];
    t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
    const uint8_t *row = table + static_cast<long long>(t) * row_bytes;
    float *o = x + static_cast<long long>(b) * dim + 32 * u;
    switch (type) {
    case ALJABR_ROCM_TYPE_Q4_0: dq_q4_0_block(row + 18LL * u, o); break;
    case ALJABR_ROCM_TYPE_Q8_0: dq_q8_0_block(row + 34LL * u, o); break;
    case ALJABR_ROCM_TYPE_Q4_K: dq_q4_k_sub(row + 144LL * (u >> 3), u & 7, o); break;
    case ALJABR_ROCM_TYPE_Q6_K:
        dq_q6_k_group(row + 210LL * (u >> 3), 2 * (u & 7), o);
        dq_q6_k_group(row + 210LL * (u >> 3), 2 * (u & 7) + 1, o + 16);
        break;
    case ALJABR_ROCM_TYPE_F16: {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(row) + 32 * u;
        const int n = dim - 32 * u < 32 ? dim - 32 * u : 32;
        for (int i = 0; i < n; ++i) o[i] = f16_bits_to_f32_exact(h[i]);
        break;
    }
    default: {
        const float *f = reinterpret_cast<const float *>(row) + 32 * u;
        const int n = dim - 32 * u < 32 ? dim - 32 * u : 32;
        for (int i = 0; i < n; ++i) o[i] = f[i];
        break;
    }
    }
}

// cache[b][h][pos[b]][d] = fp16(src[b][h*D + d]) (round to nearest even).
__global__ __launch_bounds__(kThreads) void kv_append_kernel(uint16_t *__restrict__ cache, const float *__restrict__ src,
                                                             const int *__restrict__ pos, int n_kv, int head_dim,
                                                             int cap) {
    const int b = blockIdx.y;
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n_kv * head_dim) return;
    if (pos[b] < 0 || pos[b] >= cap) return;   // outside the cache: nothing to store
    const int h = i / head_dim, d = i % head_dim;
    const _Float16 v = static_cast<_Float16>(src[static_cast<long long>(b) * n_kv * head_dim + i]);
    cache[((static_cast<long long>(b) * n_kv + h) * cap + pos[b]) * head_dim + d] = __builtin_bit_cast(uint16_t, v);
}

inline unsigned blocks_for(long long n) { return static_cast<unsigned>((n + kThreads - 1) / kThreads); }

}  // namespace

int enqueue_rmsnorm(float *out, const float *x, const float *w, int rows, int len, float eps) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kThreads), 0, current_stream(), out, x, w, rows, len, eps);
    return ALJABR_ROCM_OK;
}

int enqueue_rope(float *x, const int *pos, int rows, int n_heads, int head_dim, float base) {
    const long long total = static_cast<long long>(rows) * n_heads * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(total)), dim3(kThreads), 0, current_stream(), x, pos, rows, n_heads,
                       head_dim, base);
    return ALJABR_ROCM_OK;
}

int enqueue_swiglu(float *dst, const float *gate, const float *up, long long n) {
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for((n + 3) / 4)), dim3(kThreads), 0, current_stream(), dst, gate, up,
                       n);
    return ALJABR_ROCM_OK;
}

int enqueue_add(float *a, const float *b, long long n) {
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, current_stream(), a, b, n);
    return ALJABR_ROCM_OK;
}

int enqueue_argmax(int *out, const float *x, int rows, int cols, void *part, size_t part_bytes) {
    const int chunks = (cols + kArgmaxChunk - 1) / kArgmaxChunk;
    if (part && chunks > 1 && static_cast<size_t>(rows) * chunks * sizeof(ArgmaxPart) <= part_bytes &&
        aligned(part, 8)) {
        ArgmaxPart *pp = static_cast<ArgmaxPart *>(part);
        hipLaunchKernelGGL(argmax_chunk_kernel, dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(rows)),
                           dim3(kArgmaxThreads), 0, current_stream(), pp, x, cols);
        hipLaunchKernelGGL(argmax_final_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, current_stream(), out,
                           pp, chunks);
        return ALJABR_ROCM_OK;
    }
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(1024), 0, current_stream(), out, x, cols);
    return ALJABR_ROCM_OK;
}

size_t argmax_part_bytes(int rows, int cols) {
    return static_cast<size_t>(rows) * ((cols + kArgmaxChunk - 1) / kArgmaxChunk) * sizeof(ArgmaxPart);
}

int enqueue_embed(float *x, const float *embed, const int *tokens, int batch, int dim, int vocab) {
    const unsigned gx = static_cast<unsigned>((dim + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(embed_kernel, dim3(gx, batch), dim3(kThreads), 0, current_stream(), x, embed, tokens, dim, vocab);
    return ALJABR_ROCM_OK;
}

int enqueue_embed_typed(float *x, const void *table, int type, const int *tokens, int batch, int dim, int vocab) {
    long long row_bytes;
    switch (type) {
    case ALJABR_ROCM_TYPE_F32: row_bytes = 4LL * dim; break;
    case ALJABR_ROCM_TYPE_F16: row_bytes = 2LL * dim; break;
    case ALJABR_ROCM_TYPE_Q4_0: row_bytes = dim % 32 ? -1 : dim / 32 * 18LL; break;
    case ALJABR_ROCM_TYPE_Q8_0: row_bytes = dim % 32 ? -1 : dim / 32 * 34LL; break;
    case ALJABR_ROCM_TYPE_Q4_K: row_bytes = dim % 256 ? -1 : dim / 256 * 144LL; break;
    case ALJABR_ROCM_TYPE_Q6_K: row_bytes = dim % 256 ? -1 : dim / 256 * 210LL; break;
    default: row_bytes = -1; break;
    }
    if (row_bytes < 0) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int units = (dim + 31) / 32;
    const unsigned gx = static_cast<unsigned>((units + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(embed_typed_kernel, dim3(gx, batch), dim3(kThreads), 0, current_stream(), x,
                       static_cast<const uint8_t *>(table), type, tokens, dim, vocab, row_bytes);
    return ALJABR_ROCM_OK;
}

int enqueue_rope_append(float *q, const float *k, const float *v, uint16_t *kc, uint16_t *vc, const int *pos, int batch,
                        int nh, int nkv, int head_dim, int cap, float base, const float2 *cs) {
    if (head_dim < 2 || head_dim % 2 != 0 || head_dim / 2 > 1024) return ALJABR_ROCM_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(rope_append_kernel, dim3(nh + 2 * nkv, batch), dim3(head_dim / 2), 0, current_stream(), q, k, v,
                       kc, vc, pos, nh, nkv, head_dim, cap, base, cs);
    return ALJABR_ROCM_OK;
}

int enqueue_rope_table(float2 *cs, int cap, int head_dim, float base) {
    if (head_dim < 2 || head_dim % 2 != 0 || cap <= 0) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const long long n = static_cast<long long>(cap) * (head_dim / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       current_stream(), cs, cap, head_dim, base);
    return ALJABR_ROCM_OK;
}

int enqueue_kv_append(uint16_t *cache, const float *src, const int *pos, int batch, int n_kv, int head_dim, int cap) {
    const unsigned gx = static_cast<unsigned>((n_kv * head_dim + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(kv_append_kernel, dim3(gx, batch), dim3(kThreads), 0, current_stream(), cache, src, pos, n_kv,
                       head_dim, cap);
    return ALJABR_ROCM_OK;
}

}  // namespace aljabr

using namespace aljabr;

extern "C" {

int aljabr_rocm_rmsnorm(void *out, const void *x, const void *w, int rows, int len, float eps) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(out && x && w, "out, x and w must be non-null device pointers");
    ALJ_REQUIRE(rows > 0 && len > 0, "bad dimensions rows=%d len=%d", rows, len);
    ALJ_REQUIRE(eps >= 0.0f, "eps must be non-negative");
    enqueue_rmsnorm(static_cast<float *>(out), static_cast<const float *>(x), static_cast<const float *>(w), rows, len,
                    eps);
    return finish_launch("rmsnorm");
}

int aljabr_rocm_rope(void *x, const void *positions, int rows, int nHeads, int headDim, float base) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(x && positions, "x and positions must be non-null device pointers");
    ALJ_REQUIRE(rows > 0 && nHeads > 0 && headDim >= 2 && headDim % 2 == 0, "invalid RoPE dimensions");
    ALJ_REQUIRE(std::isfinite(base) && base > 1.0f, "RoPE frequency base must be finite and greater than one");
    enqueue_rope(static_cast<float *>(x), static_cast<const int *>(positions), rows, nHeads, headDim, base);
    return finish_launch("rope");
}

int aljabr_rocm_swiglu(void *dst, const void *gate, const void *up, long long n) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(dst && gate && up, "dst, gate and up must be non-null device pointers");
    ALJ_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return ALJABR_ROCM_OK;
    enqueue_swiglu(static_cast<float *>(dst), static_cast<const float *>(gate), static_cast<const float *>(up), n);
    return finish_launch("swiglu");
}

int aljabr_rocm_add_inplace(void *a, const void *b, long long n) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(a && b, "a and b must be non-null device pointers");
    ALJ_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return ALJABR_ROCM_OK;
    enqueue_add(static_cast<float *>(a), static_cast<const float *>(b), n);
    return finish_launch("add_inplace");
}

int aljabr_rocm_argmax(void *out_i32, const void *x, int rows, int cols) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(out_i32 && x, "out and x must be non-null device pointers");
    ALJ_REQUIRE(rows > 0 && cols > 0, "bad dimensions rows=%d cols=%d", rows, cols);
    // The chunk results in the stream's scratch, except under graph capture
    // (the scratch may not grow then): one workgroup per row instead.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusActive;
    void *part = nullptr;
    const size_t pb = argmax_part_bytes(rows, cols);
    if (cols > kArgmaxChunk && hipStreamIsCapturing(current_stream(), &cs) == hipSuccess &&
        cs == hipStreamCaptureStatusNone)
        part = stream_scratch(pb, kScratchPartials);
    enqueue_argmax(static_cast<int *>(out_i32), static_cast<const float *>(x), rows, cols, part, part ? pb : 0);
    return finish_launch("argmax");
}

}  // extern "C"
