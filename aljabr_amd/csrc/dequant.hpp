// dequant.hpp - bit-exact decoders of one quantization block (or sub-block)
// to fp32, shared by the dequantize entry point and the typed embedding
// lookup. Each multiply and add is rounded on its own (__fmul_rn, __fadd_rn,
// __fsub_rn), in the reference's order:
//   Q4_0 GRT/GgufBlockDequantizer.java:33-37,403-416  (q-8)*d + 0.0f
//   Q8_0 GRT/GgufBlockDequantizer.java:231-265        (int8)q * d
//   Q4_K GRT/GgufKBlockDequantizer.java:32-90          (d*sc)*q - dmin*min (0 for a zero min code or dmin == 0)
//   Q6_K GRT/GgufKBlockDequantizer.java:320-425        (d*scale)*(q6-32)
//   F16  GRT/GgufQuantTables.java:143-165              (canonical NaN)
#pragma once

#include "device.hpp"

namespace aljabr {

__device__ __forceinline__ float le_f16(const uint8_t *p) {
    return f16_bits_to_f32_exact(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
}

// One 18-byte Q4_0 block -> 32 values.
__device__ inline void dq_q4_0_block(const uint8_t *b, float *o) {
    const float d = le_f16(b);
    for (int j = 0; j < 16; ++j) {
        const int q = b[2 + j];
        o[j] = __fadd_rn(__fmul_rn(static_cast<float>((q & 15) - 8), d), 0.0f);
        o[16 + j] = __fadd_rn(__fmul_rn(static_cast<float>((q >> 4) - 8), d), 0.0f);
    }
}

// One 34-byte Q8_0 block -> 32 values.
__device__ inline void dq_q8_0_block(const uint8_t *b, float *o) {
    const float d = le_f16(b);
    for (int j = 0; j < 32; ++j) o[j] = __fmul_rn(static_cast<float>(static_cast<int8_t>(b[2 + j])), d);
}

// Sub-block `sub` (elements 32*sub .. +32) of a 144-byte Q4_K super-block.
__device__ inline void dq_q4_k_sub(const uint8_t *b, int sub, float *o) {
    const float d = le_f16(b);
    const float dmin = le_f16(b + 2);
    const uint8_t *sc = b + 4;
    int scale, mn;
    if (sub < 4) {
        scale = sc[sub] & 63;
        mn = sc[sub + 4] & 63;
    } else {
        scale = (sc[sub + 4] & 0x0F) | ((sc[sub - 4] >> 6) << 4);
        mn = (sc[sub + 4] >> 4) | ((sc[sub] >> 6) << 4);
    }
    const float d1 = __fmul_rn(d, static_cast<float>(scale));
    const float m1 = (dmin == 0.0f || mn == 0) ? 0.0f : __fmul_rn(dmin, static_cast<float>(mn));
    // Sub-block 2c + h: low (h = 0) or high (h = 1) nibbles of qs[32c .. 32c+32).
    const uint8_t *q = b + 16 + 32 * (sub >> 1);
    const int shift = 4 * (sub & 1);
    for (int l = 0; l < 32; ++l) o[l] = __fsub_rn(__fmul_rn(d1, static_cast<float>((q[l] >> shift) & 0x0F)), m1);
}

// Scale group g (elements 16g .. 16g+16) of a 210-byte Q6_K super-block.
__device__ inline void dq_q6_k_group(const uint8_t *b, int g, float *o) {
    const int h = g >> 3, quad = (g >> 1) & 3, l0 = 16 * (g & 1);
    const float d = le_f16(b + 208);
    const float scale = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(b[192 + g])));
    // Quadrant quad of half h: ql[64h + 32*(quad & 1) + l], nibble quad >> 1,
    // qh[32h + l] bits 2*quad.
    const uint8_t *ql = b + 64 * h + 32 * (quad & 1);
    const uint8_t *qh = b + 128 + 32 * h;
    const int nib = 4 * (quad >> 1), hs = 2 * quad;
    for (int i = 0; i < 16; ++i) {
        const int l = l0 + i;
        const int q = (((ql[l] >> nib) & 0x0F) | (((qh[l] >> hs) & 3) << 4)) - 32;
        o[i] = __fmul_rn(scale, static_cast<float>(q));
    }
}

}  // namespace aljabr
