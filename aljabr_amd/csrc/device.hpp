// device.hpp - gfx950 device helpers: wave64 DPP reductions, exact format
// conversions and the NF4 codebook.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace aljabr {

constexpr int kWave = 64;

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (nontemporal hint: weights are read once per call).
__device__ __forceinline__ u32x4 load_stream16(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// DPP-modified move: lanes outside row_mask keep `old` (0 here).
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}

// Sum within each 16-lane DPP row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    return v;
}

// Max within each 16-lane DPP row (identity -inf is never produced: every
// lane of a row is a source for the mirrors used here).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0xB1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x140, 0xf, 0xf, false)));
    return v;
}

// Full wave64 sum, returned uniformly (read from lane 63).
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += dpp_f32<0x142, 0xA>(v);  // row_bcast:15 -> rows 1 and 3
    v += dpp_f32<0x143, 0xC>(v);  // row_bcast:31 -> rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Value of lane (lane ^ MASK): DPP quad permutes for 1 and 2, ds_swizzle
// (bit mode, within 32 lanes) for 4, 8 and 16, ds_bpermute for 32.
template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (MASK == 1) return dpp_f32<0xB1>(v);      // quad_perm [1,0,3,2]
    else if constexpr (MASK == 2) return dpp_f32<0x4E>(v); // quad_perm [2,3,0,1]
    else if constexpr (MASK == 32) return __shfl_xor(v, 32);
    else return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (MASK << 10) | 0x1F));
}

// Butterfly sum of T = 2^t per-lane values (T <= 32) over the wave: stage s
// pairs each lane with lane ^ 2^s and keeps half of the values, so the whole
// reduction costs ~3T/2 + 6 operations instead of T separate wave sums. On
// return every lane holds the total of row wave_rows_index<T>(lane).
template <int MASK, int N>
__device__ __forceinline__ void fold_rows_stage(float *v, bool upper) {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float lo = v[i], hi = v[i + N / 2];
        v[i] = (upper ? hi : lo) + lane_xor<MASK>(upper ? lo : hi);
    }
}

template <int T>
__device__ __forceinline__ int wave_rows_index(int lane) {
    static_assert(T == 1 || T == 2 || T == 4 || T == 8 || T == 16 || T == 32, "T must be a power of two <= 32");
    int r = 0;
    for (int s = 0; (1 << s) < T; ++s) r = (r << 1) | ((lane >> s) & 1);
    return r;
}

template <int T>
__device__ __forceinline__ float wave_sum_rows(float (&v)[T]) {
    const int lane = threadIdx.x & 63;
    if constexpr (T >= 2) fold_rows_stage<1, T>(v, lane & 1);
    if constexpr (T >= 4) fold_rows_stage<2, T / 2>(v, lane & 2);
    if constexpr (T >= 8) fold_rows_stage<4, T / 4>(v, lane & 4);
    if constexpr (T >= 16) fold_rows_stage<8, T / 8>(v, lane & 8);
    if constexpr (T >= 32) fold_rows_stage<16, T / 16>(v, lane & 16);
    float r = v[0];
    if constexpr (T < 2) r += lane_xor<1>(r);
    if constexpr (T < 4) r += lane_xor<2>(r);
    if constexpr (T < 8) r += lane_xor<4>(r);
    if constexpr (T < 16) r += lane_xor<8>(r);
    if constexpr (T < 32) r += lane_xor<16>(r);
    r += lane_xor<32>(r);
    return r;
}

__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, not for its global loads in flight (__syncthreads also drains
// prefetched global loads, which a streaming loop cannot afford per tile).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Split-half RoPE angle of the pair (i, i + D/2), i < D/2, at position `pos`
// (GGUFVectorOps.rope :383-440): invFreq = base^(-2i/D) in double rounded to
// float, theta = pos * invFreq in float, cos and sin in double rounded to
// float.
__device__ __forceinline__ void rope_cos_sin(int pos, int i, int head_dim, float base, float &c, float &s) {
    const float exponent = -2.0f * static_cast<float>(i) / static_cast<float>(head_dim);
    const float inv_freq = static_cast<float>(pow(static_cast<double>(base), static_cast<double>(exponent)));
    const float theta = static_cast<float>(pos) * inv_freq;
    c = static_cast<float>(cos(static_cast<double>(theta)));
    s = static_cast<float>(sin(static_cast<double>(theta)));
}

// Sum of p[s * stride] over the K slices s = 0 .. slices-1 (slices >= 1),
// added in slice order, with U = 4, 8 or 16 loads in flight per trip (the
// smallest that covers the slices, 16 beyond): a trip's indices past the
// last slice re-read the last one (in bounds) and are not added. The split-K
// partial sums of a small-M GEMM are read this way by the kernel after it,
// one memory round trip per 16 slices.
__device__ __forceinline__ void slice_add(float &a, float v) { a += v; }
__device__ __forceinline__ void slice_add(float4 &a, const float4 &v) {
    a.x += v.x;
    a.y += v.y;
    a.z += v.z;
    a.w += v.w;
}

template <int U, class V>
__device__ __forceinline__ V slice_sum_u(const V *p, size_t stride, int slices) {
    V acc{};
    for (int s0 = 0; s0 < slices; s0 += U) {
        V v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) v[j] = p[static_cast<size_t>(min(s0 + j, slices - 1)) * stride];
#pragma unroll
        for (int j = 0; j < U; ++j)
            if (s0 + j < slices) slice_add(acc, v[j]);
    }
    return acc;
}

template <class V>
__device__ __forceinline__ V slice_sum(const V *p, size_t stride, int slices) {
    if (slices <= 4) return slice_sum_u<4>(p, stride, slices);
    if (slices <= 8) return slice_sum_u<8>(p, stride, slices);
    return slice_sum_u<16>(p, stride, slices);
}

// Rotation of (x0, x1) by the angle with cosine c and sine s, each product
// rounded separately.
__device__ __forceinline__ void rope_apply(float &x0, float &x1, float c, float s) {
    const float a = x0, b = x1;
    x0 = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
    x1 = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
}

// cos/sin of pair i at position p from a [cap][D/2] table of the values
// rope_cos_sin gives (filled once per model), or computed when there is no
// table or p is outside it.
__device__ __forceinline__ void rope_angle(const float2 *table, int cap, int pos, int i, int head_dim, float base,
                                           float &c, float &s) {
    if (table && pos >= 0 && pos < cap) {
        const float2 v = table[static_cast<long long>(pos) * (head_dim >> 1) + i];
        c = v.x;
        s = v.y;
    } else {
        rope_cos_sin(pos, i, head_dim, base, c, s);
    }
}

// ({hi,lo} >> shift)[31:0], shift in [0,31] (v_alignbit_b32).
__device__ __forceinline__ uint32_t funnel_shift_right(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbit(hi, lo, shift);
}

// Index (in fp16 elements) of element (m, c) of an [M][K] activation in the
// NF4 GEMM's fp16 A-fragment image: [m/16][c/64][(c%16)/8][lane
// 16*((c%64)/16) + m%16][c%8] (matmul_mfma.hip, nf4_xpack_kernel).
__device__ __forceinline__ size_t xpack_index(int m, int c, int K) {
    const size_t entry = (static_cast<size_t>(m >> 4) * (K >> 6) + (c >> 6)) * 2 + ((c >> 3) & 1);
    return (entry * 64 + 16 * ((c >> 4) & 3) + (m & 15)) * 8 + (c & 7);
}

// binary16 -> binary32 exactly as GgufQuantTables.f16ToF32Slow: integer-only,
// so the result does not depend on the FP16 denormal mode; NaN -> 0x7FC00000.
__device__ __forceinline__ float f16_bits_to_f32_exact(uint32_t h) {
    uint32_t sign = (h >> 15) & 1u, exponent = (h >> 10) & 0x1fu, mantissa = h & 0x3ffu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign << 31;
        } else {
            // value = mantissa * 2^-24: normalise the 10-bit mantissa.
            int lz = __builtin_clz(mantissa) - 21;          // shifts to bring the top bit to bit 10
            uint32_t m = (mantissa << lz) & 0x3ffu;
            uint32_t e = 113u - (uint32_t)lz;                // 127 - 14 - lz
            bits = (sign << 31) | (e << 23) | (m << 13);
        }
    } else if (exponent == 31) {
        bits = mantissa == 0 ? ((sign << 31) | 0x7f800000u) : 0x7fc00000u;
    } else {
        bits = (sign << 31) | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    return __uint_as_float(bits);
}

// Hardware binary16 -> binary32 (used in hot loops; scales are normal numbers).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// GGUFWriter.floatToHalfBits: truncate to 10 mantissa bits, add one ulp when
// the first dropped bit is set; overflow -> inf/0x7C01; tiny -> signed zero.
__device__ __forceinline__ uint32_t f32_to_f16_writer(float v) {
    uint32_t bits = __float_as_uint(v);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int exponent = (int)((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent >= 31) return sign | 0x7c00u | (mantissa == 0 ? 0u : 1u);
    if (exponent <= 0) {
        if (exponent < -10) return sign;
        uint32_t full = mantissa | 0x800000u;
        int shift = 14 - exponent;
        uint32_t hm = full >> shift;
        if ((full >> (shift - 1)) & 1u) hm += 1;
        return sign | hm;
    }
    uint32_t half = sign | ((uint32_t)exponent << 10) | (mantissa >> 13);
    if (mantissa & 0x1000u) half += 1;
    return half;
}

// java.lang.Math.round(float): floor(v + 1/2) exactly (done in double), NaN -> 0.
__device__ __forceinline__ int java_round(float v) {
    if (v != v) return 0;
    double r = floor((double)v + 0.5);
    if (r >= 2147483647.0) return 2147483647;
    if (r <= -2147483648.0) return (int)(-2147483647 - 1);
    return (int)r;
}

// NormalFloat-4 codebook, STC/DequantizationKernel.java:23-28 (16 fp32 levels).
__device__ __forceinline__ float nf4_level(int c) {
    constexpr float t[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
    return t[c];
}

// Same value without a memory read (a select chain on the lane's index), for
// kernels whose prologue must not wait on a constant-table load.
__device__ __forceinline__ float nf4_level_sel(int c) {
    constexpr float t[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
    float v = t[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) v = c == i ? t[i] : v;
    return v;
}

}  // namespace aljabr
