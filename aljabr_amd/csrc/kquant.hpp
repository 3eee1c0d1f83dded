// kquant.hpp - GGUF K-quant super-blocks (Q4_K, Q6_K) as the matvec kernels
// read them: one super-block of 256 weights is split over 8 lanes, lane j
// owning 16 "low" and 16 "high" weights that share one code byte each.
//
//   Q4_K, 144 bytes (GRT/GgufKBlockDequantizer.java:32-90,
//   GRT/GgufKQuantLayout.java:38-70): f16 d, f16 dmin, 12 bytes of 6-bit
//   scale/min codes, qs[128]. Byte 32c+l holds element 64c+l (low nibble) and
//   64c+32+l (high nibble); sub-block j = element/32 has weight
//   d*sc[j]*q - dmin*m[j] (a zero min code adds nothing). Lane j reads
//   qs[16j .. 16j+16): low elements 64(j/2) + 16(j%2) + i, high +32, sub-blocks
//   2(j/2) and 2(j/2)+1.
//
//   Q6_K, 210 bytes (GRT/GgufKBlockDequantizer.java:320-425): ql[128],
//   qh[64], int8 scales[16], f16 d at 208. ql byte 64h+l (l < 64) holds a low
//   and a high element 64 apart; the two high bits come from qh[32h + l%32]
//   at shift 2*(l/32) (low element) and 4 + 2*(l/32) (high element); element e
//   has scale scales[e/16] and weight d*scale*(q - 32). Lane j reads
//   ql[16j .. 16j+16): low elements 128(j/4) + 16(j%4) + i, high +64; qh
//   bytes 128 + 32(j/4) + 16(j%2) + i at shift 2*((j/2)%2); scales
//   8(j/4) + j%4 (low) and 8(j/4) + 4 + j%4 (high).
//
// Q6_K super-blocks are 210 bytes, so odd ones start 2 bytes off a dword: the
// loads below are unaligned (one global_load_dwordx4/x2 each; gfx950 serves
// unaligned global loads in hardware, which is how the compiler itself lowers
// a byte-aligned 16-byte memcpy for this target).
#pragma once

#include "device.hpp"

namespace aljabr {

constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2u __attribute__((ext_vector_type(2), aligned(1)));

// Element offsets (within the super-block) of lane j's first low element; the
// high run starts kQ4KHigh / kQ6KHigh later.
__device__ __forceinline__ int q4k_lo_elem(int j) { return 64 * (j >> 1) + 16 * (j & 1); }
__device__ __forceinline__ int q6k_lo_elem(int j) { return 128 * (j >> 2) + 16 * (j & 3); }
constexpr int kQ4KHigh = 32;
constexpr int kQ6KHigh = 64;

// Per-lane raw words of one super-block.
struct Q4KWords {
    u32x4 q;      // qs[16j .. 16j+16)
    u32x4 hdr;    // d | dmin << 16, then the 12 scale/min bytes
};
struct Q6KWords {
    u32x4 ql;     // ql[16j .. 16j+16)
    u32x4 qh;     // qh[32(j/4) + 16(j%2) .. +16)
    u32x2 sc;     // scales[8(j/4) .. 8(j/4)+8)
    uint32_t d;   // f16 bits
};

__device__ __forceinline__ void load_q4k(Q4KWords &w, const uint8_t *blk, int j) {
    w.q = load_stream16(blk + 16 + 16 * j);
    w.hdr = load_stream16(blk);
}

__device__ __forceinline__ void load_q6k(Q6KWords &w, const uint8_t *blk, int j) {
    const int h = j >> 2;
    w.ql = __builtin_nontemporal_load(reinterpret_cast<const u32x4u *>(blk + 16 * j));
    w.qh = __builtin_nontemporal_load(reinterpret_cast<const u32x4u *>(blk + 128 + 32 * h + 16 * (j & 1)));
    w.sc = __builtin_nontemporal_load(reinterpret_cast<const u32x2u *>(blk + 192 + 8 * h));
    w.d = __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(blk + 208));
}

// Scales of lane j's two sub-blocks: weight = dlo * q - mlo (low run),
// dhi * q - mhi (high run).
struct KScales {
    float dlo, dhi, mlo, mhi;
};

__device__ __forceinline__ KScales q4k_scales(const u32x4 &hdr, int j) {
    const float d = f16_bits_to_f32(hdr.x & 0xffffu);
    const float dmin = f16_bits_to_f32(hdr.x >> 16);
    // Sub-blocks 2c and 2c+1 (c = j/2) sit in bytes k = 2(c%2) and k+1 of
    // each scale dword; 4..7 (j >= 4) split their codes over three bytes: a
    // low nibble of the third dword and the top two bits of the first
    // (scales) or second (mins). Both cases are formed branch-free as one
    // dword of 6-bit codes per lane, so a wave runs one path.
    const uint32_t o = 16 * ((j >> 1) & 1);
    const bool split = j >= 4;
    const uint32_t sa = split ? (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u) : hdr.y;
    const uint32_t ma = split ? ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u) : hdr.z;
    const uint32_t sc0 = __builtin_amdgcn_ubfe(sa, o, 6), sc1 = __builtin_amdgcn_ubfe(sa, o + 8, 6);
    const uint32_t mn0 = __builtin_amdgcn_ubfe(ma, o, 6), mn1 = __builtin_amdgcn_ubfe(ma, o + 8, 6);
    KScales r;
    r.dlo = d * static_cast<float>(sc0);
    r.dhi = d * static_cast<float>(sc1);
    // dmin * min only where the code is non-zero (a NaN dmin with a zero
    // code adds nothing, GRT/GgufKQuantLayout.java:68-70).
    r.mlo = mn0 != 0 ? dmin * static_cast<float>(mn0) : 0.0f;
    r.mhi = mn1 != 0 ? dmin * static_cast<float>(mn1) : 0.0f;
    return r;
}

// Q6_K: the -32 offset is folded in as -32 * sum(x) by the caller.
__device__ __forceinline__ KScales q6k_scales(const Q6KWords &w, int j) {
    const float d = f16_bits_to_f32(w.d & 0xffffu);
    const int sh = 8 * (j & 3);
    KScales r;
    r.dlo = d * static_cast<float>(static_cast<int8_t>((w.sc.x >> sh) & 0xffu));
    r.dhi = d * static_cast<float>(static_cast<int8_t>((w.sc.y >> sh) & 0xffu));
    r.mlo = r.mhi = 0.0f;
    return r;
}

// Six-bit codes of lane j for one dword of ql (4 low/high element pairs):
// lo = ql low nibble | two qh bits << 4, hi = ql high nibble | two bits << 4.
__device__ __forceinline__ void q6k_codes(uint32_t ql, uint32_t qh, uint32_t qh_shift, uint32_t &lo, uint32_t &hi) {
    const uint32_t t = qh >> qh_shift;
    lo = (ql & 0x0f0f0f0fu) | ((t & 0x03030303u) << 4);
    hi = ((ql >> 4) & 0x0f0f0f0fu) | (t & 0x30303030u);
}

// Byte B of v as a float (the compiler emits one v_cvt_f32_ubyteB).
template <int B>
__device__ __forceinline__ float ubyte_f(uint32_t v) {
    return static_cast<float>((v >> (8 * B)) & 0xffu);
}

// Unscaled dots of one lane: plo = sum q_lo * xlo, phi = sum q_hi * xhi over
// the lane's 16 + 16 weights (codes as unsigned integers).
__device__ __forceinline__ void q4k_dots(const u32x4 &q, const float *xlo, const float *xhi, float &plo, float &phi) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = w[i] & 0x0f0f0f0fu, hi = (w[i] >> 4) & 0x0f0f0f0fu;
        a0 = fmaf(ubyte_f<0>(lo), xlo[4 * i + 0], a0);
        a1 = fmaf(ubyte_f<0>(hi), xhi[4 * i + 0], a1);
        a0 = fmaf(ubyte_f<1>(lo), xlo[4 * i + 1], a0);
        a1 = fmaf(ubyte_f<1>(hi), xhi[4 * i + 1], a1);
        a0 = fmaf(ubyte_f<2>(lo), xlo[4 * i + 2], a0);
        a1 = fmaf(ubyte_f<2>(hi), xhi[4 * i + 2], a1);
        a0 = fmaf(ubyte_f<3>(lo), xlo[4 * i + 3], a0);
        a1 = fmaf(ubyte_f<3>(hi), xhi[4 * i + 3], a1);
    }
    plo = a0;
    phi = a1;
}

__device__ __forceinline__ void q6k_dots(const Q6KWords &w, int j, const float *xlo, const float *xhi, float &plo,
                                         float &phi) {
    const uint32_t ql[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
    const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    const uint32_t sh = j & 2;                   // 0 for ql[64h + l], l < 32; 2 for l >= 32
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo, hi;
        q6k_codes(ql[i], qh[i], sh, lo, hi);
        a0 = fmaf(ubyte_f<0>(lo), xlo[4 * i + 0], a0);
        a1 = fmaf(ubyte_f<0>(hi), xhi[4 * i + 0], a1);
        a0 = fmaf(ubyte_f<1>(lo), xlo[4 * i + 1], a0);
        a1 = fmaf(ubyte_f<1>(hi), xhi[4 * i + 1], a1);
        a0 = fmaf(ubyte_f<2>(lo), xlo[4 * i + 2], a0);
        a1 = fmaf(ubyte_f<2>(hi), xhi[4 * i + 2], a1);
        a0 = fmaf(ubyte_f<3>(lo), xlo[4 * i + 3], a0);
        a1 = fmaf(ubyte_f<3>(hi), xhi[4 * i + 3], a1);
    }
    plo = a0;
    phi = a1;
}

// Lane contribution from the unscaled dots and the lane's activation sums.
template <bool Q6>
__device__ __forceinline__ float k_combine(const KScales &s, float plo, float phi, float sxlo, float sxhi) {
    if constexpr (Q6) return s.dlo * fmaf(-32.0f, sxlo, plo) + s.dhi * fmaf(-32.0f, sxhi, phi);
    else return (s.dlo * plo - s.mlo * sxlo) + (s.dhi * phi - s.mhi * sxhi);
}

}  // namespace aljabr
