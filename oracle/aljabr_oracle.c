/*
 * aljabr_oracle.c - CPU restatement of Aljabr's quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see aljabr_oracle.h): the checker for the HIP
 * kernels and the timed CPU baseline. Nothing under aljabr_amd/ may use it.
 *
 * Built with -ffp-contract=off so that a*b+c is a rounded multiply followed by
 * a rounded add, as Java evaluates it (Java never fuses unless Math.fma or a
 * Vector API fma() is written). Citations are file:line in andalus-ai/aljabr;
 * the path abbreviations are listed in aljabr_oracle.h.
 */
#include "aljabr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* GRT/GgufQuantTables.java:143-165. Normal numbers rebias the exponent,
 * subnormals are mantissa/1024 * 2^-14, any NaN becomes the canonical NaN. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exponent = (h >> 10) & 0x1fu;
    uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0) {
        if (mantissa == 0) return sign ? -0.0f : 0.0f;
        float value = ldexpf((float)mantissa / 1024.0f, -14);
        return sign ? -value : value;
    }
    if (exponent == 31) {
        if (mantissa == 0) return sign ? -INFINITY : INFINITY;
        return bits_to_f32(0x7fc00000u);
    }
    return bits_to_f32((sign << 31) | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* GWR/GGUFWriter.java:360-387. Truncate the fp32 mantissa to 10 bits and add
 * one ulp when the first dropped bit is set (round half away from zero in
 * magnitude); overflow maps to inf (or to 0x7C01 when any mantissa bit is set),
 * exponents below -24 flush to a signed zero. */
uint16_t orc_f32_to_f16_writer(float v) {
    uint32_t bits = f32_to_bits(v);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
    uint32_t mantissa = bits & 0x7fffffu;
    if (exponent >= 31) {
        return (uint16_t)(sign | 0x7c00u | (mantissa == 0 ? 0u : 1u));
    }
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        uint32_t full = mantissa | 0x800000u;
        int32_t shift = 14 - exponent;
        uint32_t half_mantissa = full >> shift;
        if ((full >> (shift - 1)) & 1u) half_mantissa += 1;
        return (uint16_t)(sign | half_mantissa);
    }
    uint32_t half = sign | ((uint32_t)exponent << 10) | (mantissa >> 13);
    if (mantissa & 0x1000u) half += 1;
    return (uint16_t)half;
}

/* Math.round(float): floor(a + 1/2) evaluated exactly. A float plus 0.5 is
 * exact in double for every |a| < 2^52, so the double sum has no rounding. */
int32_t orc_java_round(float v) {
    if (isnan(v)) return 0;
    double r = floor((double)v + 0.5);
    if (r >= 2147483647.0) return 2147483647;
    if (r <= -2147483648.0) return (int32_t)(-2147483647 - 1);
    return (int32_t)r;
}

/* ------------------------------------------------------------------------ */
/* threading helpers (GRT/GgufParallelConfig.java:64-73: chunks = 2*threads)  */
/* ------------------------------------------------------------------------ */

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

typedef void (*row_task)(const void *ctx, int64_t row_begin, int64_t row_end);

static void run_row_chunks(int64_t rows, int threads, row_task task, const void *ctx) {
    if (threads < 1) threads = 1;
    int64_t chunks = rows < 2LL * threads ? rows : 2LL * threads;
    if (chunks <= 1) {
        task(ctx, 0, rows);
        return;
    }
    int64_t per = rows / chunks, extra = rows % chunks;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
#endif
    for (int64_t c = 0; c < chunks; c++) {
        int64_t begin = c * per + (c < extra ? c : extra);
        int64_t end = begin + per + (c < extra ? 1 : 0);
        task(ctx, begin, end);
    }
}

/* ------------------------------------------------------------------------ */
/* NF4                                                                       */
/* ------------------------------------------------------------------------ */

/* STC/DequantizationKernel.java:23-28 (the bitsandbytes NormalFloat-4 levels). */
const float ORC_NF4_TABLE[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

/* STC/DequantizationKernel.java:84-102 */
void orc_nf4_dequant(const uint8_t *codes, const float *absmax, int64_t numel,
                     int32_t group_size, float *dst) {
    int64_t bytes = (numel + 1) / 2;
    for (int64_t j = 0; j < bytes; j++) {
        uint8_t b = codes[j];
        float s = absmax[(j * 2) / group_size];
        dst[2 * j] = ORC_NF4_TABLE[(b >> 4) & 15] * s;
        if (2 * j + 1 < numel) dst[2 * j + 1] = ORC_NF4_TABLE[b & 15] * s;
    }
}

static uint8_t nf4_nearest(float v) {
    /* Levels are sorted; pick the first level whose upper midpoint is >= v. */
    for (int c = 0; c < 15; c++) {
        float mid = (ORC_NF4_TABLE[c] + ORC_NF4_TABLE[c + 1]) * 0.5f;
        if (v <= mid) return (uint8_t)c;
    }
    return 15;
}

void orc_nf4_quantize(const float *w, int64_t numel, int32_t group_size,
                      uint8_t *codes, float *absmax) {
    int64_t groups = (numel + group_size - 1) / group_size;
    for (int64_t g = 0; g < groups; g++) {
        int64_t begin = g * group_size, end = begin + group_size;
        if (end > numel) end = numel;
        float m = 0.0f;
        for (int64_t i = begin; i < end; i++) {
            float a = fabsf(w[i]);
            if (a > m) m = a;
        }
        absmax[g] = m;
    }
    memset(codes, 0, (size_t)((numel + 1) / 2));
    for (int64_t i = 0; i < numel; i++) {
        float m = absmax[i / group_size];
        uint8_t c = m == 0.0f ? 7 : nf4_nearest(w[i] / m);
        if ((i & 1) == 0) codes[i >> 1] |= (uint8_t)(c << 4);
        else codes[i >> 1] |= c;
    }
}

/* 16-lane fp32 dot with a pairwise lane reduction. */
static float dot16(const float *a, const float *b, int64_t n) {
    float lanes[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; l++) lanes[l] += a[i + l] * b[i + l];
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; l++) lanes[l] += lanes[l + w];
    float r = lanes[0];
    for (; i < n; i++) r += a[i] * b[i];
    return r;
}

typedef struct {
    const uint8_t *codes; const float *absmax; int32_t group;
    const float *x; int64_t n, k; int32_t m; float *y;
} nf4_mv_ctx;

static void nf4_mv_rows(const void *vctx, int64_t r0, int64_t r1) {
    const nf4_mv_ctx *c = (const nf4_mv_ctx *)vctx;
    float *row = (float *)malloc((size_t)c->k * sizeof(float));
    for (int64_t n = r0; n < r1; n++) {
        int64_t flat = n * c->k;
        /* Dequantize the row exactly as the flat-matrix decode would. */
        for (int64_t kk = 0; kk < c->k; kk++) {
            int64_t e = flat + kk;
            uint8_t b = c->codes[e >> 1];
            int code = (e & 1) ? (b & 15) : (b >> 4);
            row[kk] = ORC_NF4_TABLE[code] * c->absmax[e / c->group];
        }
        for (int32_t mm = 0; mm < c->m; mm++)
            c->y[(int64_t)mm * c->n + n] = dot16(row, c->x + (int64_t)mm * c->k, c->k);
    }
    free(row);
}

void orc_nf4_matvec(const uint8_t *codes, const float *absmax, int32_t group_size,
                    const float *x, int64_t n_rows, int64_t k_cols, int32_t m,
                    float *y, int threads) {
    nf4_mv_ctx c = {codes, absmax, group_size, x, n_rows, k_cols, m, y};
    run_row_chunks(n_rows, threads, nf4_mv_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* GGUF Q4_0 / Q8_0                                                          */
/* ------------------------------------------------------------------------ */

static float max_abs(const float *v, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(v[i]);
        m = a > m ? a : m;
    }
    return m;
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void put_le16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)(v & 0xff); p[1] = (uint8_t)(v >> 8); }
static uint16_t get_le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* GWR/GGUFWriter.java:179-209: fp32 scale = maxAbs/7 is used to quantize, the
 * fp16 (writer rounding) copy is stored; byte i = (hi+8)<<4 | (lo+8) with lo
 * from element i and hi from element 16+i. */
void orc_q4_0_quantize(const float *w, int64_t numel, uint8_t *out) {
    for (int64_t blk = 0; blk < numel / 32; blk++) {
        const float *v = w + blk * 32;
        uint8_t *o = out + blk * 18;
        float scale = max_abs(v, 32) / 7.0f;
        put_le16(o, orc_f32_to_f16_writer(scale));
        for (int i = 0; i < 16; i++) {
            int lo = scale == 0.0f ? 0 : clampi(orc_java_round(v[i] / scale), -8, 7);
            int hi = scale == 0.0f ? 0 : clampi(orc_java_round(v[16 + i] / scale), -8, 7);
            o[2 + i] = (uint8_t)(((hi + 8) << 4) | (lo + 8));
        }
    }
}

/* GWR/GGUFWriter.java:163-177 */
void orc_q8_0_quantize(const float *w, int64_t numel, uint8_t *out) {
    for (int64_t blk = 0; blk < numel / 32; blk++) {
        const float *v = w + blk * 32;
        uint8_t *o = out + blk * 34;
        float scale = max_abs(v, 32) / 127.0f;
        put_le16(o, orc_f32_to_f16_writer(scale));
        for (int i = 0; i < 32; i++) {
            int q = scale == 0.0f ? 0 : orc_java_round(v[i] / scale);
            o[2 + i] = (uint8_t)(clampi(q, -127, 127) & 0xff);
        }
    }
}

/* GRT/GgufBlockDequantizer.java:33-37 with bias 0.0f and zero point 8,
 * :366-416 lane order. */
void orc_q4_0_dequant(const uint8_t *blocks, int64_t numel, float *dst) {
    for (int64_t blk = 0; blk < numel / 32; blk++) {
        const uint8_t *b = blocks + blk * 18;
        float d = orc_f16_to_f32(get_le16(b));
        float *o = dst + blk * 32;
        for (int j = 0; j < 16; j++) {
            int q = b[2 + j];
            o[j] = (float)((q & 15) - 8) * d + 0.0f;
            o[16 + j] = (float)((q >> 4) - 8) * d + 0.0f;
        }
    }
}

/* GRT/GgufBlockDequantizer.java:231-265 */
void orc_q8_0_dequant(const uint8_t *blocks, int64_t numel, float *dst) {
    for (int64_t blk = 0; blk < numel / 32; blk++) {
        const uint8_t *b = blocks + blk * 34;
        float d = orc_f16_to_f32(get_le16(b));
        for (int j = 0; j < 32; j++) dst[blk * 32 + j] = (float)(int8_t)b[2 + j] * d;
    }
}

/* GRT/GgufQ32RawDot.java:454-463: one packed byte contributes its low nibble
 * against x[index] and its high nibble against x[16+index]. */
static inline float q4_pair(const uint8_t *q, int index, const float *x) {
    int b = q[index];
    return (float)((b & 15) - 8) * x[index] + (float)((b >> 4) - 8) * x[16 + index];
}

/* GRT/GgufQ32RawDot.java:428-450: four partials over bytes {i, i+4, i+8, i+12}. */
static float q4_0_unscaled_block(const uint8_t *q, const float *x) {
    float s0 = q4_pair(q, 0, x) + q4_pair(q, 4, x) + q4_pair(q, 8, x) + q4_pair(q, 12, x);
    float s1 = q4_pair(q, 1, x) + q4_pair(q, 5, x) + q4_pair(q, 9, x) + q4_pair(q, 13, x);
    float s2 = q4_pair(q, 2, x) + q4_pair(q, 6, x) + q4_pair(q, 10, x) + q4_pair(q, 14, x);
    float s3 = q4_pair(q, 3, x) + q4_pair(q, 7, x) + q4_pair(q, 11, x) + q4_pair(q, 15, x);
    return s0 + s1 + s2 + s3;
}

/* GRT/GgufQ32RawDot.java:342-349 */
static float q4_0_block(const uint8_t *blk, const float *x) {
    return orc_f16_to_f32(get_le16(blk)) * q4_0_unscaled_block(blk + 2, x);
}

/* GRT/GgufQ32RawDot.java:34-67 */
float orc_q4_0_dot_row(const uint8_t *row, int32_t columns, const float *x) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int blocks = columns / 32, b = 0;
    for (; b <= blocks - 4; b += 4) {
        s0 += q4_0_block(row + (b + 0) * 18, x + (b + 0) * 32);
        s1 += q4_0_block(row + (b + 1) * 18, x + (b + 1) * 32);
        s2 += q4_0_block(row + (b + 2) * 18, x + (b + 2) * 32);
        s3 += q4_0_block(row + (b + 3) * 18, x + (b + 3) * 32);
    }
    float sum = s0 + s1 + s2 + s3;
    for (; b < blocks; b++) sum += q4_0_block(row + b * 18, x + b * 32);
    return sum;
}

/* GRT/GgufQ8RawDot.java:784-830: four partials over byte lanes {i, i+4, ...}
 * combined two products at a time. */
static float q8_unscaled_block(const uint8_t *q, const float *x) {
    float s[4];
    for (int lane = 0; lane < 4; lane++) {
        float acc = (float)(int8_t)q[lane] * x[lane] + (float)(int8_t)q[lane + 4] * x[lane + 4];
        for (int base = 8; base < 32; base += 8)
            acc += (float)(int8_t)q[base + lane] * x[base + lane]
                   + (float)(int8_t)q[base + lane + 4] * x[base + lane + 4];
        s[lane] = acc;
    }
    return s[0] + s[1] + s[2] + s[3];
}

/* GRT/GgufQ8RawDot.java:138-185 */
float orc_q8_0_dot_row(const uint8_t *row, int32_t columns, const float *x) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int blocks = columns / 32, b = 0;
    for (; b <= blocks - 4; b += 4) {
        for (int u = 0; u < 4; u++) {
            const uint8_t *blk = row + (b + u) * 34;
            float v = orc_f16_to_f32(get_le16(blk)) * q8_unscaled_block(blk + 2, x + (b + u) * 32);
            if (u == 0) s0 += v; else if (u == 1) s1 += v; else if (u == 2) s2 += v; else s3 += v;
        }
    }
    float sum = s0 + s1 + s2 + s3;
    for (; b < blocks; b++) {
        const uint8_t *blk = row + b * 34;
        sum += orc_f16_to_f32(get_le16(blk)) * q8_unscaled_block(blk + 2, x + b * 32);
    }
    return sum;
}

/* ---- GGUF K-quants: Q4_K (144-byte super-blocks of 256) and Q6_K (210) ---- */

/* GRT/GgufKQuantLayout.java:38-66: 6-bit scale and min codes of sub-block
 * idx (0..7) from the 12 packed bytes. */
static void q4_k_scale_min(const uint8_t *s, int idx, int *sc, int *mn) {
    if (idx < 4) {
        *sc = s[idx] & 63;
        *mn = s[idx + 4] & 63;
    } else {
        *sc = (s[idx + 4] & 0x0F) | ((s[idx - 4] >> 6) << 4);
        *mn = (s[idx + 4] >> 4) | ((s[idx] >> 6) << 4);
    }
}

/* GRT/GgufKBlockDequantizer.java:32-90 with GRT/GgufKQuantLayout.java:68-70
 * (a zero min code contributes 0 whatever dMin holds, NaN included). */
void orc_q4_k_dequant(const uint8_t *blocks, int64_t numel, float *dst) {
    for (int64_t blk = 0; blk < numel / 256; blk++) {
        const uint8_t *b = blocks + blk * 144;
        const float d = orc_f16_to_f32(get_le16(b));
        const float dmin = orc_f16_to_f32(get_le16(b + 2));
        const uint8_t *q = b + 16;
        float *o = dst + blk * 256;
        for (int j = 0; j < 4; j++) {
            int sc1, mn1, sc2, mn2;
            q4_k_scale_min(b + 4, 2 * j, &sc1, &mn1);
            q4_k_scale_min(b + 4, 2 * j + 1, &sc2, &mn2);
            const float d1 = d * (float)sc1, d2 = d * (float)sc2;
            float m1 = 0.0f, m2 = 0.0f;
            if (dmin != 0.0f) {
                m1 = mn1 == 0 ? 0.0f : dmin * (float)mn1;
                m2 = mn2 == 0 ? 0.0f : dmin * (float)mn2;
            }
            for (int l = 0; l < 32; l++) {
                o[64 * j + l] = d1 * (float)(q[32 * j + l] & 0x0F) - m1;
                o[64 * j + 32 + l] = d2 * (float)(q[32 * j + l] >> 4) - m2;
            }
        }
    }
}

/* GRT/GgufKBlockDequantizer.java:320-425: ql[128] low nibbles, qh[64] two-bit
 * high parts, int8 scales[16], f16 d at byte 208; element e of half h
 * (128 elements) takes scale index 8h + (e % 128) / 16. */
void orc_q6_k_dequant(const uint8_t *blocks, int64_t numel, float *dst) {
    for (int64_t blk = 0; blk < numel / 256; blk++) {
        const uint8_t *b = blocks + blk * 210;
        const float d = orc_f16_to_f32(get_le16(b + 208));
        float *o = dst + blk * 256;
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
            const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const float s1 = d * (float)sc[is], s2 = d * (float)sc[is + 2];
                const float s3 = d * (float)sc[is + 4], s4 = d * (float)sc[is + 6];
                const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[32 + l] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[128 * h + l] = s1 * (float)q1;
                o[128 * h + 32 + l] = s2 * (float)q2;
                o[128 * h + 64 + l] = s3 * (float)q3;
                o[128 * h + 96 + l] = s4 * (float)q4;
            }
        }
    }
}

/* GRT/GgufQ4RawDot.java:38-148 (dotRowQ4K): per 64-element chunk, integer
 * nibble dots against x accumulated eight products at a time, then
 * d1*dot1 + d2*dot2 and, for non-zero min codes of a block with dMin != 0,
 * - dMin*min*sum(x). */
float orc_q4_k_dot_row(const uint8_t *row, int32_t columns, const float *x) {
    float sum = 0.0f;
    for (int blk = 0; blk < columns / 256; blk++) {
        const uint8_t *b = row + (int64_t)blk * 144;
        const float *v = x + (int64_t)blk * 256;
        const float d = orc_f16_to_f32(get_le16(b));
        const float dmin = orc_f16_to_f32(get_le16(b + 2));
        const int has_mins = dmin != 0.0f;
        const uint8_t *q = b + 16;
        for (int j = 0; j < 4; j++) {
            int sc1, mn1, sc2, mn2;
            q4_k_scale_min(b + 4, 2 * j, &sc1, &mn1);
            q4_k_scale_min(b + 4, 2 * j + 1, &sc2, &mn2);
            if (!has_mins) mn1 = mn2 = 0;
            const float d1 = d * (float)sc1, d2 = d * (float)sc2;
            float vs1 = 0.0f, vs2 = 0.0f, qd1 = 0.0f, qd2 = 0.0f;
            const float *v1 = v + 64 * j, *v2 = v + 64 * j + 32;
            for (int i = 0; i < 32; i += 8) {
                float t1 = 0.0f, t2 = 0.0f, u1 = 0.0f, u2 = 0.0f;
                for (int e = 0; e < 8; e++) {
                    const int qb = q[32 * j + i + e];
                    const float p1 = (float)(qb & 0x0F) * v1[i + e];
                    const float p2 = (float)(qb >> 4) * v2[i + e];
                    t1 = e == 0 ? p1 : t1 + p1;
                    t2 = e == 0 ? p2 : t2 + p2;
                    u1 = e == 0 ? v1[i + e] : u1 + v1[i + e];
                    u2 = e == 0 ? v2[i + e] : u2 + v2[i + e];
                }
                qd1 += t1;
                qd2 += t2;
                if (mn1 != 0) vs1 += u1;
                if (mn2 != 0) vs2 += u2;
            }
            sum += d1 * qd1 + d2 * qd2;
            if (mn1 != 0) sum -= dmin * (float)mn1 * vs1;
            if (mn2 != 0) sum -= dmin * (float)mn2 * vs2;
        }
    }
    return sum;
}

/* GRT/GgufQ6RawDot.java:403-514 (dotRowQ6KHalf): 16 elements per quadrant,
 * quadrant dots scaled by d*scale and summed. */
static float q6_k_half(const uint8_t *ql, const uint8_t *qh, const float *v, int off, float s1, float s2,
                       float s3, float s4) {
    float qd1 = 0.0f, qd2 = 0.0f, qd3 = 0.0f, qd4 = 0.0f;
    for (int i = off; i < off + 16; i += 8) {
        float t1 = 0.0f, t2 = 0.0f, t3 = 0.0f, t4 = 0.0f;
        for (int e = 0; e < 8; e++) {
            const int l = i + e;
            const float p1 = (float)(((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32) * v[l];
            const float p2 = (float)(((ql[32 + l] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32) * v[32 + l];
            const float p3 = (float)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32) * v[64 + l];
            const float p4 = (float)(((ql[32 + l] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32) * v[96 + l];
            t1 = e == 0 ? p1 : t1 + p1;
            t2 = e == 0 ? p2 : t2 + p2;
            t3 = e == 0 ? p3 : t3 + p3;
            t4 = e == 0 ? p4 : t4 + p4;
        }
        qd1 += t1;
        qd2 += t2;
        qd3 += t3;
        qd4 += t4;
    }
    return s1 * qd1 + s2 * qd2 + s3 * qd3 + s4 * qd4;
}

/* GRT/GgufQ6RawDot.java:77-133 (one super-block: four half sums). */
static float q6_k_block(const uint8_t *b, const float *v) {
    const float d = orc_f16_to_f32(get_le16(b + 208));
    const int8_t *sc = (const int8_t *)(b + 192);
    float s[4];
    for (int part = 0; part < 4; part++) {
        const int h = part >> 1, off = (part & 1) * 16, base = 8 * h + (part & 1);
        s[part] = q6_k_half(b + 64 * h, b + 128 + 32 * h, v + 128 * h, off, d * (float)sc[base],
                            d * (float)sc[base + 2], d * (float)sc[base + 4], d * (float)sc[base + 6]);
    }
    return s[0] + s[1] + s[2] + s[3];
}

/* GRT/GgufQ6RawDot.java:33-75 (dotRowQ6K: four block accumulators). */
float orc_q6_k_dot_row(const uint8_t *row, int32_t columns, const float *x) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    const int blocks = columns / 256;
    int b = 0;
    for (; b <= blocks - 4; b += 4) {
        s0 += q6_k_block(row + (int64_t)(b + 0) * 210, x + (int64_t)(b + 0) * 256);
        s1 += q6_k_block(row + (int64_t)(b + 1) * 210, x + (int64_t)(b + 1) * 256);
        s2 += q6_k_block(row + (int64_t)(b + 2) * 210, x + (int64_t)(b + 2) * 256);
        s3 += q6_k_block(row + (int64_t)(b + 3) * 210, x + (int64_t)(b + 3) * 256);
    }
    float sum = s0 + s1 + s2 + s3;
    for (; b < blocks; b++) sum += q6_k_block(row + (int64_t)b * 210, x + (int64_t)b * 256);
    return sum;
}

typedef struct {
    const uint8_t *w; const float *x; int64_t n, k; int32_t m; float *y; int type;
} q_mv_ctx;

static void q_mv_rows(const void *vctx, int64_t r0, int64_t r1) {
    const q_mv_ctx *c = (const q_mv_ctx *)vctx;
    int64_t row_bytes = c->type == 12 ? (c->k / 256) * 144
                      : c->type == 14 ? (c->k / 256) * 210
                                      : (c->k / 32) * (c->type == 2 ? 18 : 34);
    for (int64_t n = r0; n < r1; n++) {
        const uint8_t *row = c->w + n * row_bytes;
        for (int32_t mm = 0; mm < c->m; mm++) {
            const float *x = c->x + (int64_t)mm * c->k;
            float v;
            switch (c->type) {
            case 2: v = orc_q4_0_dot_row(row, (int32_t)c->k, x); break;
            case 12: v = orc_q4_k_dot_row(row, (int32_t)c->k, x); break;
            case 14: v = orc_q6_k_dot_row(row, (int32_t)c->k, x); break;
            default: v = orc_q8_0_dot_row(row, (int32_t)c->k, x); break;
            }
            c->y[(int64_t)mm * c->n + n] = v;
        }
    }
}

void orc_q4_0_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads) {
    q_mv_ctx c = {w, x, n_rows, k_cols, m, y, 2};
    run_row_chunks(n_rows, threads, q_mv_rows, &c);
}

void orc_q8_0_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads) {
    q_mv_ctx c = {w, x, n_rows, k_cols, m, y, 8};
    run_row_chunks(n_rows, threads, q_mv_rows, &c);
}

void orc_q4_k_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads) {
    q_mv_ctx c = {w, x, n_rows, k_cols, m, y, 12};
    run_row_chunks(n_rows, threads, q_mv_rows, &c);
}

void orc_q6_k_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads) {
    q_mv_ctx c = {w, x, n_rows, k_cols, m, y, 14};
    run_row_chunks(n_rows, threads, q_mv_rows, &c);
}

/* Output soft cap of aljabr_metal_matvec_tb_q4_k_softcap / _q6_k_softcap
 * (MTLC/aljabr_metal_matvec_api.m:448-505 with aljabr_softcap_kernel,
 * MTLC/aljabr_metal_kernel_source.m:111-118): y = cap * tanh(y / cap). */
void orc_softcap(float *y, int64_t n, float cap) {
    for (int64_t i = 0; i < n; i++) y[i] = cap * (float)tanh((double)(y[i] / cap));
}

/* GRT/GgufDenseDot.java:289-320: element i of the unrolled body feeds
 * accumulator i % 4; the four are summed, then the tail is added. */
static float f16_dot_row(const uint16_t *row, int64_t k, const float *x) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t i = 0;
    for (; i + 16 <= k; i += 16)
        for (int j = 0; j < 16; j++) s[j & 3] += orc_f16_to_f32(row[i + j]) * x[i + j];
    float sum = s[0] + s[1] + s[2] + s[3];
    for (; i < k; i++) sum += orc_f16_to_f32(row[i]) * x[i];
    return sum;
}

typedef struct { const uint16_t *w; const float *x; int64_t n, k; int32_t m; float *y; } f16_mv_ctx;

static void f16_mv_rows(const void *vctx, int64_t r0, int64_t r1) {
    const f16_mv_ctx *c = (const f16_mv_ctx *)vctx;
    for (int64_t n = r0; n < r1; n++)
        for (int32_t mm = 0; mm < c->m; mm++)
            c->y[(int64_t)mm * c->n + n] = f16_dot_row(c->w + n * c->k, c->k, c->x + (int64_t)mm * c->k);
}

void orc_f16_matvec(const uint16_t *w, const float *x, int64_t n_rows,
                    int64_t k_cols, int32_t m, float *y, int threads) {
    f16_mv_ctx c = {w, x, n_rows, k_cols, m, y};
    run_row_chunks(n_rows, threads, f16_mv_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

/* CPU/CpuBackend.java:1668-1748 for one (batch, query head) group. */
static void attention_group(const float *q, const float *k, const float *v,
                            const float *mask, float *out, int64_t group,
                            int64_t key_group, int64_t sq, int64_t sk, int64_t d,
                            float scale, int causal, double *weighted) {
    int64_t q_base = group * sq * d;
    int64_t k_base = key_group * sk * d;
    for (int64_t qi = 0; qi < sq; qi++) {
        for (int64_t j = 0; j < d; j++) weighted[j] = 0.0;
        float running_max = -INFINITY;
        double denominator = 0.0;
        int64_t causal_limit = sk - sq + qi;
        int64_t key_limit = causal ? (sk < causal_limit + 1 ? sk : causal_limit + 1) : sk;
        for (int64_t ki = 0; ki < key_limit; ki++) {
            float additive = mask ? mask[qi * sk + ki] : 0.0f;
            if (additive == -INFINITY) continue;
            float score = dot16(q + q_base + qi * d, k + k_base + ki * d, d) * scale + additive;
            float next_max;
            double previous_scale, current_scale;
            if (isfinite(score)) {
                if (score > running_max) {
                    previous_scale = exp((double)(running_max - score));
                    current_scale = 1.0;
                    next_max = score;
                } else {
                    previous_scale = 1.0;
                    current_scale = exp((double)(score - running_max));
                    next_max = running_max;
                }
            } else {
                next_max = running_max > score ? running_max : score;
                if (isnan(running_max) || isnan(score)) next_max = NAN;
                previous_scale = running_max == -INFINITY ? 0.0 : exp((double)(running_max - next_max));
                current_scale = exp((double)(score - next_max));
            }
            denominator = denominator * previous_scale + current_scale;
            for (int64_t j = 0; j < d; j++)
                weighted[j] = weighted[j] * previous_scale + current_scale * (double)v[k_base + ki * d + j];
            running_max = next_max;
        }
        for (int64_t j = 0; j < d; j++)
            out[q_base + qi * d + j] = denominator == 0.0 ? 0.0f : (float)(weighted[j] / denominator);
    }
}

int orc_attention_gqa(const float *q, const float *k, const float *v,
                      const float *mask, int64_t b, int64_t hq, int64_t hkv,
                      int64_t sq, int64_t sk, int64_t d, int causal,
                      float *out, int threads) {
    /* CPU/CpuBackend.java:1566-1587 shape and mask validation. */
    if (b <= 0 || hq <= 0 || hkv <= 0 || sq <= 0 || sk <= 0 || d <= 0 || hq % hkv != 0) return -2;
    if (mask) {
        for (int64_t i = 0; i < sq * sk; i++)
            if (isnan(mask[i]) || mask[i] == INFINITY) return -2;
    }
    float scale = (float)(1.0 / sqrt((double)d));
    int64_t groups = b * hq;
    int64_t per_kv = hq / hkv;
    (void)threads;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
    {
        double *weighted = (double *)malloc((size_t)d * sizeof(double));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t g = 0; g < groups; g++) {
            int64_t head = g % hq;
            int64_t kv_head = head / per_kv;
            attention_group(q, k, v, mask, out, g, (g / hq) * hkv + kv_head, sq, sk, d,
                            scale, causal, weighted);
        }
        free(weighted);
    }
    return 0;
}

/* FA4 prefill attention as the Metal backend's fallback computes it
 * (MTLC/aljabr_metal_fa4.m:466-530): per (b, h) the scores scale * q.k over
 * all S keys, keys from the causal limit on excluded
 * (causal_limit_for_row, :111-115), the soft cap cap * tanh(s / cap) on the
 * kept scores, softmax by exp(s - max) / sum, then the weighted sum of V rows.
 * Sums are carried in double. */
int orc_fa4_attention(const float *q, const float *k, const float *v, int32_t b_n, int32_t t_n, int32_t s_n,
                      int32_t h_n, int32_t hkv, int32_t d, float scale, int32_t is_causal, float soft_cap,
                      int32_t window, float *out) {
    if (b_n <= 0 || t_n <= 0 || s_n <= 0 || h_n <= 0 || hkv <= 0 || d <= 0 || h_n % hkv != 0) return -1;
    int32_t group = h_n / hkv;
    float *row = (float *)malloc((size_t)s_n * sizeof(float));
    double *acc = (double *)malloc((size_t)d * sizeof(double));
    if (!row || !acc) {
        free(row);
        free(acc);
        return -1;
    }
    for (int32_t b = 0; b < b_n; b++)
        for (int32_t h = 0; h < h_n; h++) {
            int32_t kvh = h / group;
            for (int32_t t = 0; t < t_n; t++) {
                const float *qr = q + (((int64_t)b * t_n + t) * h_n + h) * d;
                float *orow = out + (((int64_t)b * t_n + t) * h_n + h) * d;
                int32_t hi = s_n;
                if (is_causal) {
                    int32_t lim = (s_n > t_n ? s_n - t_n : 0) + t + 1;
                    hi = lim < s_n ? lim : s_n;
                }
                int32_t lo = 0;
                if (window > 0) lo = hi - window > 0 ? hi - window : 0;
                float mx = -INFINITY;
                for (int32_t s = lo; s < hi; s++) {
                    const float *kr = k + (((int64_t)b * s_n + s) * hkv + kvh) * d;
                    double dot = 0.0;
                    for (int32_t e = 0; e < d; e++) dot += (double)qr[e] * kr[e];
                    float sc = (float)dot * scale;
                    if (soft_cap > 0.0f) sc = soft_cap * tanhf(sc / soft_cap);
                    row[s] = sc;
                    if (sc > mx) mx = sc;
                }
                double sum = 0.0;
                for (int32_t e = 0; e < d; e++) acc[e] = 0.0;
                for (int32_t s = lo; s < hi; s++) {
                    double p = exp((double)row[s] - (double)mx);
                    sum += p;
                    const float *vr = v + (((int64_t)b * s_n + s) * hkv + kvh) * d;
                    for (int32_t e = 0; e < d; e++) acc[e] += p * vr[e];
                }
                for (int32_t e = 0; e < d; e++) orow[e] = sum > 0.0 ? (float)(acc[e] / sum) : 0.0f;
            }
        }
    free(row);
    free(acc);
    return 0;
}

/* Paged-KV attention of the Metal bridge's CPU path
 * (MTLC/aljabr_metal_attention.m:146-160 resolve_attention_bounds, :162-355
 * aljabr_metal_attention_impl): Q/out [B,T,H,D], caches [phys][H_kv][bs][D]
 * through block_table[b*max_blocks + blk]; float scores dot*scale, optional
 * soft cap, exp(s - max), weights * 1/(sum + 1e-9), float weighted V sums. */
int orc_paged_attention(const float *q, const float *kc, const float *vc, const int32_t *block_table,
                        const int32_t *context_lens, int32_t b_n, int32_t t_n, int32_t h_n, int32_t hkv,
                        int32_t d, int32_t block_size, int32_t max_blocks, float scale, int32_t is_causal,
                        int32_t query_start_pos, int32_t sliding_window, float soft_cap, float *out) {
    if (hkv <= 0 || h_n % hkv != 0) return -1;
    if (b_n <= 0 || t_n <= 0 || h_n <= 0 || d <= 0 || block_size <= 0 || max_blocks <= 0) return -2;
    int32_t group = h_n / hkv;
    for (int32_t b = 0; b < b_n; b++) {
        int32_t ctx = context_lens[b];
        float *bo = out + (int64_t)b * t_n * h_n * d;
        if (ctx <= 0) {
            memset(bo, 0, (size_t)t_n * h_n * d * sizeof(float));
            continue;
        }
        int32_t nblk = (ctx + block_size - 1) / block_size;
        if (nblk > max_blocks) return -2;
        for (int32_t blk = 0; blk < nblk; blk++)
            if (block_table[(int64_t)b * max_blocks + blk] < 0) return -2;
        float *row = (float *)malloc((size_t)ctx * sizeof(float));
        for (int32_t h = 0; h < h_n; h++) {
            int32_t kvh = h / group;
            for (int32_t t = 0; t < t_n; t++) {
                const float *qh = q + (((int64_t)b * t_n + t) * h_n + h) * d;
                float *oh = bo + ((int64_t)t * h_n + h) * d;
                int32_t qpos = query_start_pos;
                if (is_causal && sliding_window <= 0 && query_start_pos == 0 && ctx >= t_n) qpos = ctx - t_n;
                int32_t abs_pos = qpos + t;
                int32_t upper = is_causal ? abs_pos : ctx - 1;
                if (upper >= ctx) upper = ctx - 1;
                int32_t lower = sliding_window > 0 ? abs_pos - sliding_window + 1 : 0;
                if (lower < 0) lower = 0;
                memset(oh, 0, (size_t)d * sizeof(float));
                if (upper < lower) continue;
                float mx = -1e30f;
                for (int32_t s = lower; s <= upper; s++) {
                    int64_t phys = block_table[(int64_t)b * max_blocks + s / block_size];
                    const float *kh = kc + ((phys * hkv + kvh) * block_size + s % block_size) * d;
                    float dot = 0.0f;
                    for (int32_t e = 0; e < d; e++) dot += qh[e] * kh[e];
                    float score = dot * scale;
                    if (soft_cap > 0.0f) score = soft_cap * tanhf(score / soft_cap);
                    row[s] = score;
                    if (score > mx) mx = score;
                }
                float sum = 0.0f;
                for (int32_t s = lower; s <= upper; s++) {
                    row[s] = expf(row[s] - mx);
                    sum += row[s];
                }
                float inv = 1.0f / (sum + 1e-9f);
                for (int32_t s = lower; s <= upper; s++) row[s] *= inv;
                for (int32_t s = lower; s <= upper; s++) {
                    int64_t phys = block_table[(int64_t)b * max_blocks + s / block_size];
                    const float *vh = vc + ((phys * hkv + kvh) * block_size + s % block_size) * d;
                    for (int32_t e = 0; e < d; e++) oh[e] += row[s] * vh[e];
                }
            }
        }
        free(row);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* decode-step element-wise ops                                              */
/* ------------------------------------------------------------------------ */

/* GLD/tensor/GGUFVectorOps.java:211-234: fused-multiply-add sum of squares in
 * vector lanes (16 here), 1/sqrt in double, then (x * scale) * w. */
void orc_rmsnorm(const float *x, const float *w, float *out, int32_t len, float eps) {
    float lanes[16] = {0};
    int32_t i = 0;
    for (; i + 16 <= len; i += 16)
        for (int l = 0; l < 16; l++) lanes[l] = fmaf(x[i + l], x[i + l], lanes[l]);
    for (int s = 8; s >= 1; s >>= 1)
        for (int l = 0; l < s; l++) lanes[l] += lanes[l + s];
    float ss = lanes[0];
    for (; i < len; i++) ss += x[i] * x[i];
    float scale = 1.0f / (float)sqrt((double)(ss / (float)len + eps));
    for (int32_t j = 0; j < len; j++) out[j] = (x[j] * scale) * w[j];
}

/* GLD/tensor/GGUFVectorOps.java:383-440 (no frequency factors, full rotary). */
void orc_rope(float *x, int32_t n_heads, int32_t head_dim, int32_t pos, float base) {
    int32_t half = head_dim / 2;
    float *table = (float *)malloc((size_t)head_dim * sizeof(float));
    for (int32_t i = 0; i < half; i++) {
        float exponent = -2.0f * (float)i / (float)head_dim;
        float inv_freq = (float)pow((double)base, (double)exponent);
        float theta = ((float)pos * inv_freq) / 1.0f;
        table[i] = (float)cos((double)theta);
        table[half + i] = (float)sin((double)theta);
    }
    for (int32_t h = 0; h < n_heads; h++) {
        float *p = x + (int64_t)h * head_dim;
        for (int32_t i = 0; i < half; i++) {
            float c = table[i], s = table[half + i];
            float x0 = p[i], x1 = p[i + half];
            p[i] = x0 * c - x1 * s;
            p[i + half] = x0 * s + x1 * c;
        }
    }
    free(table);
}

/* GLD/tensor/GGUFVectorOps.java:333-338 */
void orc_swiglu(const float *gate, const float *up, float *dst, int32_t len) {
    for (int32_t i = 0; i < len; i++) {
        float g = gate[i] / (1.0f + (float)exp(-(double)gate[i]));
        dst[i] = g * up[i];
    }
}

/* GLD/tensor/GGUFVectorOps.java:302-317 */
void orc_softmax(float *a, int32_t len) {
    float mx = a[0];
    for (int32_t i = 1; i < len; i++) if (a[i] > mx) mx = a[i];
    float sum = 0.0f;
    for (int32_t i = 0; i < len; i++) {
        a[i] = (float)exp((double)(a[i] - mx));
        sum += a[i];
    }
    float inv = 1.0f / sum;
    for (int32_t i = 0; i < len; i++) a[i] *= inv;
}

/* ------------------------------------------------------------------------ */
/* Llama-shaped decode step                                                  */
/* ------------------------------------------------------------------------ */

/* Single-token GQA attention over a position-major cache window, the decode
 * runner's attention (GJB/GgufDecodeAttentionExecution.java:68-104): keys and
 * values are [position][cache_head_stride], KV head h at offset h * head_dim;
 * query head h reads KV head h / (query_heads / kv_heads); positions
 * [start_position, sequence_length) are visible. Scores are the dot times
 * `scale`, GGUFVectorOps.softmax normalises them (max, exp, 1/sum), and the
 * value rows are added in position order (scaledAddInPlace). `scores` holds
 * sequence_length - start_position floats. */
void orc_decode_attention(const float *query, float *output, float *scores, const float *key_cache,
                          const float *value_cache, int32_t cache_head_stride, int32_t kv_heads,
                          int32_t query_heads, int32_t head_dim, int32_t sequence_length,
                          int32_t start_position, float scale) {
    const int32_t active = sequence_length - start_position;
    for (int64_t i = 0; i < (int64_t)query_heads * head_dim; i++) output[i] = 0.0f;
    for (int32_t h = 0; h < query_heads; h++) {
        const int32_t kvh = h / (query_heads / kv_heads);
        const float *q = query + (int64_t)h * head_dim;
        for (int32_t p = start_position; p < sequence_length; p++)
            scores[p - start_position] =
                dot16(q, key_cache + (int64_t)p * cache_head_stride + (int64_t)kvh * head_dim, head_dim) * scale;
        orc_softmax(scores, active);
        float *o = output + (int64_t)h * head_dim;
        for (int32_t p = start_position; p < sequence_length; p++) {
            const float *vr = value_cache + (int64_t)p * cache_head_stride + (int64_t)kvh * head_dim;
            const float s = scores[p - start_position];
            for (int32_t j = 0; j < head_dim; j++) o[j] += s * vr[j];
        }
    }
}

/* y[n] = sum_k W[n][k] x[k] for one typed matrix (GgufDecodePass's per-type
 * row dots: GRT/GgufMatVec.java:27-97 dispatching on the GgmlType). */
static void typed_mv(const orc_tensor *t, const float *x, int64_t n, int64_t k, float *y, int threads) {
    switch (t->type) {
    case 100: orc_nf4_matvec((const uint8_t *)t->data, t->absmax, t->group, x, n, k, 1, y, threads); break;
    case 2: orc_q4_0_matvec((const uint8_t *)t->data, x, n, k, 1, y, threads); break;
    case 8: orc_q8_0_matvec((const uint8_t *)t->data, x, n, k, 1, y, threads); break;
    case 12: orc_q4_k_matvec((const uint8_t *)t->data, x, n, k, 1, y, threads); break;
    case 14: orc_q6_k_matvec((const uint8_t *)t->data, x, n, k, 1, y, threads); break;
    case 1: orc_f16_matvec((const uint16_t *)t->data, x, n, k, 1, y, threads); break;
    default: {                                   /* F32 rows */
        const float *w = (const float *)t->data;
        for (int64_t r = 0; r < n; r++) y[r] = dot16(w + r * k, x, k);
        break;
    }
    }
}

/* Row `row` of a typed [rows][dim] table decoded to fp32 (the embedding
 * lookup: GgufDecodeStep's token_embd row dequantization). */
static void typed_row(const orc_tensor *t, int64_t row, int64_t dim, float *out) {
    switch (t->type) {
    case 1: {
        const uint16_t *h = (const uint16_t *)t->data + row * dim;
        for (int64_t i = 0; i < dim; i++) out[i] = orc_f16_to_f32(h[i]);
        break;
    }
    case 2: orc_q4_0_dequant((const uint8_t *)t->data + row * (dim / 32) * 18, dim, out); break;
    case 8: orc_q8_0_dequant((const uint8_t *)t->data + row * (dim / 32) * 34, dim, out); break;
    case 12: orc_q4_k_dequant((const uint8_t *)t->data + row * (dim / 256) * 144, dim, out); break;
    case 14: orc_q6_k_dequant((const uint8_t *)t->data + row * (dim / 256) * 210, dim, out); break;
    default: memcpy(out, (const float *)t->data + row * dim, (size_t)dim * 4); break;
    }
}

int32_t orc_llama_decode_typed(const orc_llama_cfg *cfg, const orc_llama_typed *w,
                               int32_t token, int32_t pos, float *k_cache,
                               float *v_cache, float *logits, float *hidden,
                               int threads) {
    const int32_t dim = cfg->dim, hd = cfg->head_dim, nh = cfg->n_heads, nkv = cfg->n_kv_heads;
    const int32_t kvd = nkv * hd, qd = nh * hd, ffn = cfg->ffn;
    float *x = hidden;
    float *xb = (float *)malloc((size_t)dim * 4), *q = (float *)malloc((size_t)qd * 4);
    float *kk = (float *)malloc((size_t)kvd * 4), *vv = (float *)malloc((size_t)kvd * 4);
    float *att = (float *)malloc((size_t)qd * 4), *scores = (float *)malloc((size_t)(pos + 1) * 4);
    float *gate = (float *)malloc((size_t)ffn * 4), *up = (float *)malloc((size_t)ffn * 4);
    float *hb = (float *)malloc((size_t)ffn * 4);
    typed_row(&w->tok_embed, token, dim, x);
    float scale = (float)(1.0 / sqrt((double)hd));
    for (int32_t l = 0; l < cfg->layers; l++) {
        orc_rmsnorm(x, w->attn_norm[l], xb, dim, cfg->eps);
        typed_mv(&w->wq[l], xb, qd, dim, q, threads);
        typed_mv(&w->wk[l], xb, kvd, dim, kk, threads);
        typed_mv(&w->wv[l], xb, kvd, dim, vv, threads);
        orc_rope(q, nh, hd, pos, cfg->rope_base);
        orc_rope(kk, nkv, hd, pos, cfg->rope_base);
        float *kc = k_cache + (int64_t)l * cfg->max_seq * kvd;
        float *vc = v_cache + (int64_t)l * cfg->max_seq * kvd;
        for (int32_t j = 0; j < kvd; j++) {
            kc[(int64_t)pos * kvd + j] = cfg->kv_f16 ? orc_round_f16(kk[j]) : kk[j];
            vc[(int64_t)pos * kvd + j] = cfg->kv_f16 ? orc_round_f16(vv[j]) : vv[j];
        }
        /* GgufDecodePass's attention: every cached position 0..pos, no window. */
        orc_decode_attention(q, att, scores, kc, vc, kvd, nkv, nh, hd, pos + 1, 0, scale);
        typed_mv(&w->wo[l], att, dim, qd, xb, threads);
        for (int32_t j = 0; j < dim; j++) x[j] += xb[j];
        orc_rmsnorm(x, w->ffn_norm[l], xb, dim, cfg->eps);
        typed_mv(&w->w_gate[l], xb, ffn, dim, gate, threads);
        typed_mv(&w->w_up[l], xb, ffn, dim, up, threads);
        orc_swiglu(gate, up, hb, ffn);
        typed_mv(&w->w_down[l], hb, dim, ffn, xb, threads);
        for (int32_t j = 0; j < dim; j++) x[j] += xb[j];
    }
    orc_rmsnorm(x, w->out_norm, xb, dim, cfg->eps);
    typed_mv(&w->lm_head, xb, cfg->vocab, dim, logits, threads);
    int32_t best = 0;
    for (int32_t i = 1; i < cfg->vocab; i++) if (logits[i] > logits[best]) best = i;
    free(xb); free(q); free(kk); free(vv); free(att); free(scores); free(gate); free(up); free(hb);
    return best;
}

/* The NF4 layout (fp32 embedding, NF4 projections, fp16 LM head) through the
 * typed step. */
int32_t orc_llama_decode(const orc_llama_cfg *cfg, const orc_llama_weights *w,
                         int32_t token, int32_t pos, float *k_cache,
                         float *v_cache, float *logits, float *hidden,
                         int threads) {
    const int32_t L = cfg->layers, g = cfg->nf4_group;
    orc_tensor *t = (orc_tensor *)malloc(sizeof(orc_tensor) * 7 * (size_t)L);
    for (int32_t l = 0; l < L; l++) {
        const orc_tensor q = {w->wq[l], w->wq_s[l], 100, g}, k = {w->wk[l], w->wk_s[l], 100, g};
        const orc_tensor v = {w->wv[l], w->wv_s[l], 100, g}, o = {w->wo[l], w->wo_s[l], 100, g};
        const orc_tensor ga = {w->w_gate[l], w->w_gate_s[l], 100, g}, u = {w->w_up[l], w->w_up_s[l], 100, g};
        const orc_tensor d = {w->w_down[l], w->w_down_s[l], 100, g};
        t[0 * L + l] = q; t[1 * L + l] = k; t[2 * L + l] = v; t[3 * L + l] = o;
        t[4 * L + l] = ga; t[5 * L + l] = u; t[6 * L + l] = d;
    }
    orc_llama_typed tw;
    const orc_tensor emb = {w->tok_embed, NULL, 0, 0}, lm = {w->lm_head, NULL, 1, 0};
    tw.tok_embed = emb;
    tw.attn_norm = w->attn_norm;
    tw.ffn_norm = w->ffn_norm;
    tw.wq = t; tw.wk = t + L; tw.wv = t + 2 * L; tw.wo = t + 3 * L;
    tw.w_gate = t + 4 * L; tw.w_up = t + 5 * L; tw.w_down = t + 6 * L;
    tw.out_norm = w->out_norm;
    tw.lm_head = lm;
    const int32_t r = orc_llama_decode_typed(cfg, &tw, token, pos, k_cache, v_cache, logits, hidden, threads);
    free(t);
    return r;
}

/* ------------------------------------------------------------------------ */
/* Metal whole-step decode (registered layers)                               */
/* ------------------------------------------------------------------------ */

/* act(gate) * up of the Metal FFN kernels (MTLC/aljabr_metal_kernel_source.m:
 * 72-108): SiLU g / (1 + e^-g) with 0 at or below -20 and g at or above 20,
 * or for kind 2 the tanh GELU with 0 at or below -10 and g at or above 10; a
 * non-finite product becomes 0. */
static void metal_gated_act(const float *gate, const float *up, float *out, int32_t n, int32_t kind) {
    for (int32_t i = 0; i < n; i++) {
        const float g = gate[i];
        float act;
        if (kind == 2) {
            if (g <= -10.0f) act = 0.0f;
            else if (g >= 10.0f) act = g;
            else act = 0.5f * g * (1.0f + (float)tanh((double)(0.79788456f * (g + 0.044715f * g * g * g))));
        } else {
            if (g <= -20.0f) act = 0.0f;
            else if (g >= 20.0f) act = g;
            else act = g / (1.0f + (float)exp(-(double)g));
        }
        const float y = act * up[i];
        out[i] = isfinite(y) ? y : 0.0f;
    }
}

/* rows of `len`: x * 1/sqrt(mean(x^2) + eps) (* w when w is not NULL), the
 * Metal rmsnorm_rows / rmsnorm_unit_rows kernels (MTLC/aljabr_metal_kernel_
 * source.m:482-547) with addOne = 0. */
static void metal_norm_rows(float *x, const float *w, int32_t rows, int32_t len, float eps) {
    for (int32_t r = 0; r < rows; r++) {
        float *p = x + (int64_t)r * len;
        double ss = 0.0;
        for (int32_t i = 0; i < len; i++) ss += (double)p[i] * p[i];
        const float inv = (float)(1.0 / sqrt(ss / len + eps));
        for (int32_t i = 0; i < len; i++) p[i] = w ? (p[i] * inv) * w[i] : p[i] * inv;
    }
}

/* Split-half RoPE of `heads` rows at `pos`: freq = base^(-2i/D), theta =
 * pos * freq / ff with ff = factors[i] when that is positive (the
 * rope_freqs divisors) else 1; MTLC/aljabr_metal_kernel_source.m:845-884. */
static void metal_rope(float *x, int32_t heads, int32_t hd, int32_t pos, float base, const float *factors,
                       int32_t nfactors) {
    const int32_t half = hd / 2;
    for (int32_t i = 0; i < half; i++) {
        const double freq = 1.0 / pow((double)base, 2.0 * i / (double)hd);
        const float ff = (factors && i < nfactors) ? factors[i] : 1.0f;
        const double theta = (double)pos * freq / (ff > 0.0f ? (double)ff : 1.0);
        const float c = (float)cos(theta), s = (float)sin(theta);
        for (int32_t h = 0; h < heads; h++) {
            float *p = x + (int64_t)h * hd;
            const float x0 = p[i], x1 = p[i + half];
            p[i] = x0 * c - x1 * s;
            p[i + half] = x0 * s + x1 * c;
        }
    }
}

static int tensor_present(const orc_tensor *t) { return t->data != NULL; }

/* MTLC/aljabr_metal_matvec_api.m:3222-3266 (KV owner resolution) and
 * :3574-4083 (aljabr_metal_decode_step_internal), one position: */
int32_t orc_step_decode(const orc_step_model *m, int32_t pos, int32_t window, float eps, int32_t token,
                        const float *x_in, float *x, float *logits, int threads) {
    if (m->layers <= 0) return -1;
    const orc_step_layer *L0 = &m->layer[0];
    const int32_t dim = L0->wo_n;
    int32_t max_q = 0, max_kv = 0, max_att = 0, max_ffn = 0, max_hd = 0;
    for (int32_t l = 0; l < m->layers; l++) {
        const orc_step_layer *c = &m->layer[l];
        if (c->n0 > max_q) max_q = c->n0;
        if (c->n1 > max_kv) max_kv = c->n1;
        if (c->n2 > max_kv) max_kv = c->n2;
        if (c->wo_k > max_att) max_att = c->wo_k;
        if (c->ffn > max_ffn) max_ffn = c->ffn;
        if (c->head_dim > max_hd) max_hd = c->head_dim;
    }
    if (!m->norm[1] || !m->norm[3]) return -3;            /* ffn and attn norms are required */
    /* the input: an embedding row (decode_step_token) or x_in */
    if (token >= 0) {
        if (!tensor_present(&m->embd) || token >= m->embd_rows) return -6;
        typed_row(&m->embd, token, dim, x);
        if (m->embd_scale != 1.0f)
            for (int32_t i = 0; i < dim; i++) x[i] *= m->embd_scale;
    } else {
        if (!x_in) return -5;
        memcpy(x, x_in, (size_t)dim * 4);
    }
    float *xb = (float *)calloc((size_t)(dim > max_att ? dim : max_att), 4);
    float *q = (float *)calloc((size_t)max_q + 1, 4), *kk = (float *)calloc((size_t)max_kv + 1, 4);
    float *vv = (float *)calloc((size_t)max_kv + 1, 4), *att = (float *)calloc((size_t)max_att + 1, 4);
    float *scores = (float *)calloc((size_t)pos + 1, 4), *gate = (float *)calloc((size_t)max_ffn, 4);
    float *up = (float *)calloc((size_t)max_ffn, 4), *hb = (float *)calloc((size_t)max_ffn, 4);
    int32_t rc = 0;
    for (int32_t l = 0; l < m->layers && rc == 0; l++) {
        const orc_step_layer *c = &m->layer[l];
        const int32_t hd = c->head_dim;
        const int has_k = tensor_present(&c->wk), has_v = tensor_present(&c->wv);
        orc_rmsnorm(x, m->norm[3] + (int64_t)l * dim, xb, dim, eps);          /* attn norm, slot 3 */
        typed_mv(&c->wq, xb, c->n0, dim, q, threads);
        if (has_k) typed_mv(&c->wk, xb, c->n1, dim, kk, threads);
        if (has_v) typed_mv(&c->wv, xb, c->n2, dim, vv, threads);
        if (has_k && !has_v) {                                              /* K as V: the raw projection */
            if (c->n1 <= 0 || c->n1 != c->n2) { rc = -6; break; }
            memcpy(vv, kk, (size_t)c->n1 * 4);
        }
        if (c->has_q_norm && m->norm[4]) metal_norm_rows(q, m->norm[4] + (int64_t)l * max_hd, c->n_heads, hd, eps);
        if (c->has_k_norm && m->norm[5] && has_k)
            metal_norm_rows(kk, m->norm[5] + (int64_t)l * max_hd, c->n_kv_heads, hd, eps);
        if (c->has_unit_v_norm && (has_k || has_v)) metal_norm_rows(vv, NULL, c->n_kv_heads, hd, eps);
        metal_rope(q, c->n_heads, hd, pos, c->freq_base, c->rope_freqs, c->rope_freqs_len);
        if (has_k) metal_rope(kk, c->n_kv_heads, hd, pos, c->freq_base, c->rope_freqs, c->rope_freqs_len);
        if (has_k && m->k_cache[l] && m->v_cache[l]) {                     /* this layer owns a cache */
            const int32_t kvw = c->n_kv_heads * hd;                       /* stride >= kvw */
            memcpy(m->k_cache[l] + (int64_t)pos * m->kv_stride[l], kk, (size_t)kvw * 4);
            memcpy(m->v_cache[l] + (int64_t)pos * m->kv_stride[l], vv, (size_t)kvw * 4);
        }
        /* the KV owner: follow kv_layer links to a layer with a K projection */
        int32_t owner = c->kv_layer, hops = 0;
        while (owner >= 0 && owner < m->layers && hops++ < m->layers) {
            const orc_step_layer *cand = &m->layer[owner];
            if (tensor_present(&cand->wk) || cand->kv_layer == owner) break;
            owner = cand->kv_layer;
        }
        if (owner < 0 || owner >= m->layers || !m->k_cache[owner] || !m->v_cache[owner] ||
            !tensor_present(&m->layer[owner].wk)) { rc = -4; break; }
        const orc_step_layer *oc = &m->layer[owner];
        if (oc->head_dim != hd || oc->n_kv_heads != c->n_kv_heads || m->kv_stride[owner] < c->n_kv_heads * hd) {
            rc = -5;
            break;
        }
        const int32_t seq = pos + 1;
        const int32_t start = (c->is_swa && window > 0 && seq > window) ? seq - window : 0;
        float scale = c->attn_scale;
        if (scale <= 0.0f) scale = (c->has_q_norm || c->has_k_norm) ? 1.0f : (float)(1.0 / sqrt((double)hd));
        orc_decode_attention(q, att, scores, m->k_cache[owner], m->v_cache[owner], m->kv_stride[owner],
                             oc->n_kv_heads, c->n_heads, hd, seq, start, scale);
        typed_mv(&c->wo, att, dim, c->wo_k, xb, threads);
        if (c->has_post_attn_norm && m->norm[0]) metal_norm_rows(xb, m->norm[0] + (int64_t)l * dim, 1, dim, eps);
        for (int32_t i = 0; i < dim; i++) x[i] += xb[i];
        orc_rmsnorm(x, m->norm[1] + (int64_t)l * dim, xb, dim, eps);           /* ffn norm, slot 1 */
        typed_mv(&c->gate, xb, c->ffn, dim, gate, threads);
        typed_mv(&c->up, xb, c->ffn, dim, up, threads);
        metal_gated_act(gate, up, hb, c->ffn, m->activation);
        typed_mv(&c->down, hb, dim, c->ffn, xb, threads);
        if (c->has_post_ffn_norm && m->norm[2]) metal_norm_rows(xb, m->norm[2] + (int64_t)l * dim, 1, dim, eps);
        const int scale_out = c->out_scale > 0.0f && c->out_scale != 1.0f;
        for (int32_t i = 0; i < dim; i++) {
            const float v = x[i] + xb[i];
            x[i] = scale_out ? v * c->out_scale : v;
        }
    }
    int32_t best = 0;
    if (rc == 0 && tensor_present(&m->out_w) && m->out_norm) {
        orc_rmsnorm(x, m->out_norm, xb, m->out_k, eps);
        typed_mv(&m->out_w, xb, m->out_n, m->out_k, logits, threads);
        if (m->cap > 0.0f) orc_softcap(logits, m->out_n, m->cap);
        for (int32_t i = 1; i < m->out_n; i++) if (logits[i] > logits[best]) best = i;
    }
    free(xb); free(q); free(kk); free(vv); free(att); free(scores); free(gate); free(up); free(hb);
    return rc ? rc : best;
}

float orc_round_f16(float v) {
    uint32_t b = f32_to_bits(v);
    uint32_t sign = b & 0x80000000u;
    uint32_t a = b & 0x7fffffffu;
    if (a >= 0x7f800000u) return v;                      /* inf / nan unchanged */
    float f = bits_to_f32(a);
    float r;
    if (f >= 65520.0f) {
        r = INFINITY;                                    /* rounds past the largest half */
    } else if (f < 6.103515625e-05f) {
        /* subnormal half: quantum 2^-24; nearbyint rounds half to even */
        r = (float)(nearbyint((double)f * 16777216.0) / 16777216.0);
    } else {
        int e;
        frexpf(f, &e);                                   /* f = m * 2^e, m in [0.5, 1) */
        double q = ldexp(1.0, e - 11);                   /* half ulp spacing at this binade */
        r = (float)(nearbyint((double)f / q) * q);
    }
    return bits_to_f32(f32_to_bits(r) | sign);
}

/* ------------------------------------------------------------------------ */
/* generator                                                                 */
/* ------------------------------------------------------------------------ */

static inline uint64_t splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double unit_open(uint64_t *state) {
    /* (0, 1]: never zero, so log() is finite. */
    return ((double)(splitmix64(state) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(uint64_t seed, float mean, float std, float *out, int64_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    int64_t i = 0;
    for (; i + 1 < n; i += 2) {
        double r = sqrt(-2.0 * log(unit_open(&state)));
        double t = two_pi * unit_open(&state);
        out[i] = (float)(mean + std * r * cos(t));
        out[i + 1] = (float)(mean + std * r * sin(t));
    }
    if (i < n) {
        double r = sqrt(-2.0 * log(unit_open(&state)));
        double t = two_pi * unit_open(&state);
        out[i] = (float)(mean + std * r * cos(t));
    }
}

void orc_fill_uniform_int(uint64_t seed, int32_t bound, int32_t *out, int64_t n) {
    uint64_t state = seed;
    for (int64_t i = 0; i < n; i++) out[i] = (int32_t)(splitmix64(&state) % (uint64_t)bound);
}
