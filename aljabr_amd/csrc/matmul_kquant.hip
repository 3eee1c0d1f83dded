// matmul_kquant.hip - GGUF small-M GEMM on the matrix cores for the block
// formats Q4_K, Q6_K, Q4_0 and Q8_0: Y[M,N] = X[M,K] . W[N,K]^T for
// 2 <= M <= 32 per pass (a decode batch). W is read from HBM once for all M
// tokens.
//
// MFMA v_mfma_f32_32x32x16_f16 with fp32 accumulation. A = X split into two
// fp16 parts, x = hi + lo (hi = fp16(x), lo = fp16(x - hi)): each B fragment
// is multiplied by both, which carries x to ~2^-22 instead of fp16's 2^-11.
// B = W^T (32 weight rows per wave as the output columns) holds small exact
// integers in fp16; every fp16/fp32 block scale stays fp32 on the accumulators:
//   Q4_K  B = q * sc (q <= 15, sc <= 63: <= 945, exact), one MFMA pair per
//         32-element sub-block; the min term sum_s dmin * m_s * sum(x in s)
//         is one more MFMA pair per super-block, A = the split per-sub-block
//         sums of x, B = the 6-bit min codes; then C += d * C_q - dmin * C_min.
//   Q6_K  the int8 scale splits as sc = sl + (sc - sl), sl = sc & 15, so
//         B_lo = (q - 32) * sl (|.| <= 480) and B_hi = (q - 32) * (sc - sl)
//         (16 times an integer of |.| <= 256) are both exact in fp16; per
//         16-element scale group x_hi meets B_lo and B_hi and x_lo their
//         fp16 sum (whose rounding, 2^-12 of B, is scaled by x_lo ~ 2^-11 x);
//         C += d * C_q.
//   Q4_0  B = q - 8, Q8_0 B = q; per 32-element block C += d * C_b, where
//         C_b is the block's two MFMA steps (x hi and lo each). These run
//         2 <= M <= 8 tokens per pass, so only the accumulators of rows
//         m < 8 (four per lane) are scaled.
// Codes become fp16 integers with v_perm against a constant 0x64 byte: the
// half 0x64qq is 1024 + qq exactly. Q4_K low nibbles give 1024 + q, high
// nibbles (masked in place) 1024 + 16q, and one packed fp16 FMA removes the
// offset and applies the scale without rounding: (1024 + q) * sc - 1024 * sc,
// (1024 + 16q) * (sc/16) - 64 * sc. Q6_K: (1024 + q) - 1056, then * scale.
// Q4_0: (1024 + q) - 1032 and (1024 + 16q) / 16 - 72; Q8_0 bytes are biased
// by xor 0x80 and (1024 + q + 128) - 1152.
//
// Operand layout (32x32x16): lane l supplies A[m = l%32][8*(l/32) + e] and
// B[8*(l/32) + e][n = l%32]; accumulator r is C[8*(r/4) + 4*(l/32) + r%4][l%32].
// One MFMA step covers 16 consecutive elements of a row, lane half h the 8
// at 8h: for Q4_K sub-block s = 2c + t (t: low/high nibbles of qs[32c ..
// 32c+32)) step j reads qs[32c + 16j + 8h .. +8]; for Q6_K group g (elements
// 16g .. 16g+15) reads the ql/qh bytes of those elements; Q4_0 block b reads
// qs[8h .. 8h+8) once for both steps (low nibbles: elements 0..15, high:
// 16..31); Q8_0 step j reads qs[16j + 8h .. +8].
//
// Work split as the NF4 kernel: a workgroup is 8 waves x 32 rows and one
// K-slice of KS elements; a work unit is the wave's 32 rows x 256 elements
// (one K-quant super-block, eight Q4_0/Q8_0 blocks: 144, 210, 144 and 272
// bytes a row). Weights are loaded coalesced (whole row segments per lane
// group) and transposed through per-wave LDS rows, two units ahead. With
// several K-slices each stores its partial tile and enqueue_slice_sum adds
// the slices in order (deterministic: no float atomics).
#include <algorithm>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"
#include "kquant.hpp"

namespace aljabr {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowsPerWg = kWaves * 32;

// Up to three weight matrices of the same type and K stacked as one row
// space (the decode step's Q/K/V or gate/up in one launch): segment s owns
// stacked rows [end[s-1], end[s]); all but the last hold a multiple of 32
// rows, so a wave's 32-row tile never straddles two.
struct KqArgs {
    float *y[3];
    const float *x;
    const uint8_t *w[3];
    int end[3];
    int nseg;
    int M, N, K;   // N: stacked rows
    int add;       // one K slice: Y += instead of Y =
    float *part;   // several K slices: partial sums part[slice][m][col0 + stacked row], row stride ld
    int ld, col0;
    int groups, slices;   // row groups (kRowsPerWg * NT rows each) and K slices of the launch
};

// The segment of the tile starting at stacked row r0.
struct KqTile {
    const uint8_t *w;
    float *y;
    int local0, n;
};

__device__ __forceinline__ KqTile kq_tile(const KqArgs &a, int r0) {
    int s = (r0 >= a.end[0]) + (r0 >= a.end[1]);
    if (s > a.nseg - 1) s = a.nseg - 1;
    const int start = s == 0 ? 0 : s == 1 ? a.end[0] : a.end[1];
    KqTile t;
    t.w = s == 0 ? a.w[0] : s == 1 ? a.w[1] : a.w[2];
    t.y = s == 0 ? a.y[0] : s == 1 ? a.y[1] : a.y[2];
    t.local0 = r0 - start;
    t.n = (s == 0 ? a.end[0] : s == 1 ? a.end[1] : a.end[2]) - start;
    return t;
}

// Row formats of the kernel.
enum : int { kFQ4K = 0, kFQ6K = 1, kFQ40 = 2, kFQ80 = 3 };

template <int F> struct KqGeom {
    // Bytes of a row's 256-element unit, its 16-byte pieces (Q6_K: 13 + the
    // 2-byte d) and the staging row stride (8-byte aligned; an odd number of
    // 8-byte words, so 32 rows' 8-byte reads hit distinct banks).
    static constexpr int BB = F == kFQ4K ? kQ4KBytes : F == kFQ6K ? kQ6KBytes : F == kFQ40 ? 8 * 18 : 8 * 34;
    static constexpr int SEGS = F == kFQ4K ? 9 : F == kFQ6K ? 14 : F == kFQ40 ? 9 : 17;
    static constexpr int STR = F == kFQ4K ? 152 : F == kFQ6K ? 216 : F == kFQ40 ? 152 : 280;
    static constexpr int LOADS = (32 * SEGS + 63) / 64;
};

__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
    const _Float16 a = static_cast<_Float16>(lo), b = static_cast<_Float16>(hi);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

__device__ __forceinline__ uint32_t pk_fma_exact(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2v, a),
                                                                  __builtin_bit_cast(half2v, b),
                                                                  __builtin_bit_cast(half2v, c)));
}

// Halves 0x64bb from bytes 2i and 2i+1 of `w`: v_perm against a constant
// 0x64 byte (selector values 0-3 pick bytes of w, 4 the constant).
template <int I>
__device__ __forceinline__ uint32_t magic_pair(uint32_t w) {
    constexpr uint32_t b0 = 2 * I, b1 = 2 * I + 1;
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04000400u | (b1 << 16) | b0);
}

// B fragment of 8 codes held one per byte in (w0, w1) as 0x64qq halves,
// mapped by one packed fp16 FMA each: v * mul + add.
__device__ __forceinline__ half8 fma_frag(uint32_t w0, uint32_t w1, uint32_t mul2, uint32_t add2) {
    u32x4v r;
    r.x = pk_fma_exact(magic_pair<0>(w0), mul2, add2);
    r.y = pk_fma_exact(magic_pair<1>(w0), mul2, add2);
    r.z = pk_fma_exact(magic_pair<0>(w1), mul2, add2);
    r.w = pk_fma_exact(magic_pair<1>(w1), mul2, add2);
    return __builtin_bit_cast(half8, r);
}

// Six-bit codes (one per byte of w0, w1) -> (q - 32) * sl, (q - 32) * sh16
// (both exact) and their fp16 sum.
__device__ __forceinline__ void q6_frags(uint32_t w0, uint32_t w1, uint32_t sl2, uint32_t sh2, half8 &blo, half8 &bhi,
                                         half8 &bsum) {
    constexpr uint32_t kMinus1056 = 0xE420E420u;     // fp16 -1056 in both halves
    const uint32_t p[4] = {magic_pair<0>(w0), magic_pair<1>(w0), magic_pair<0>(w1), magic_pair<1>(w1)};
    u32x4v lo, hi, sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v v = __builtin_bit_cast(half2v, p[i]) + __builtin_bit_cast(half2v, kMinus1056);
        const half2v a = v * __builtin_bit_cast(half2v, sl2), b = v * __builtin_bit_cast(half2v, sh2);
        lo[i] = __builtin_bit_cast(uint32_t, a);
        hi[i] = __builtin_bit_cast(uint32_t, b);
        sum[i] = __builtin_bit_cast(uint32_t, a + b);
    }
    blo = __builtin_bit_cast(half8, lo);
    bhi = __builtin_bit_cast(half8, hi);
    bsum = __builtin_bit_cast(half8, sum);
}

// fp16 bits of a small integer in both halves, times `mul` (a power of two).
__device__ __forceinline__ uint32_t int_half2(int v, float mul) {
    const _Float16 h = static_cast<_Float16>(static_cast<float>(v) * mul);
    const uint32_t b = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
    return b | (b << 16);
}

__device__ __forceinline__ uint32_t half_bits(float v) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v)));
}

template <int F, int KS>
constexpr size_t kq_lds_bytes() {
    // x slice split in two fp16 parts (2 x [32][KS+8]) + Q4_K sub-block sums
    // (2 x [32][KS/32+8]) + per-wave staging rows.
    return 2 * (static_cast<size_t>(32) * (KS + 8) * 2 + (F != kFQ4K ? 0 : static_cast<size_t>(32) * (KS / 32 + 8) * 2)) +
           static_cast<size_t>(kWaves) * 32 * KqGeom<F>::STR;
}

// Eight bytes at LDS byte address p, where p % 4 == al (0 or 2; a constant
// once the caller's loops are unrolled), as two words.
__device__ __forceinline__ void lds_bytes8(const uint8_t *p, int al, uint32_t &w0, uint32_t &w1) {
    if (al == 0) {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
        w0 = q[0];
        w1 = q[1];
    } else {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(p - 2);
        const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
        w0 = __builtin_amdgcn_alignbyte(d1, d0, 2);
        w1 = __builtin_amdgcn_alignbyte(d2, d1, 2);
    }
}

// Coalesced loads of one unit (the wave's 32 rows x one super-block): piece
// p = 64i + lane is 16-byte segment p % SEGS of row p / SEGS (Q6_K: the last
// piece is bytes 194..209, read for its last two bytes, d, so that no load
// leaves the block).
template <int F>
__device__ __forceinline__ void issue_unit(u32x4 (&q)[KqGeom<F>::LOADS], const KqArgs &a, const KqTile &tr, int sb,
                                           int lane) {
    using G = KqGeom<F>;
    const size_t row_bytes = static_cast<size_t>(a.K >> 8) * G::BB;
#pragma unroll
    for (int i = 0; i < G::LOADS; ++i) {
        const int p = min(64 * i + lane, 32 * G::SEGS - 1);
        const int r = p / G::SEGS, seg = p - r * G::SEGS;
        const int row = min(tr.local0 + r, tr.n - 1);
        const uint8_t *src = tr.w + static_cast<size_t>(row) * row_bytes + static_cast<size_t>(sb) * G::BB + 16 * seg;
        if constexpr (F == kFQ6K) {
            q[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4u *>(seg == G::SEGS - 1 ? src - 14 : src));
        } else {
            q[i] = load_stream16(src);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

template <int F>
__device__ __forceinline__ void stage_unit(uint8_t *st, const u32x4 (&q)[KqGeom<F>::LOADS], int lane) {
    using G = KqGeom<F>;
#pragma unroll
    for (int i = 0; i < G::LOADS; ++i) {
        const int p = 64 * i + lane;
        if (p < 32 * G::SEGS) {
            const int r = p / G::SEGS, seg = p - r * G::SEGS;
            uint8_t *dst = st + r * G::STR + 16 * seg;
            if (F == kFQ6K && seg == G::SEGS - 1) {
                *reinterpret_cast<uint16_t *>(dst) = static_cast<uint16_t>(q[i].w >> 16);   // d at 208
            } else {
                *reinterpret_cast<u32x2v *>(dst) = u32x2v{q[i].x, q[i].y};
                *reinterpret_cast<u32x2v *>(dst + 8) = u32x2v{q[i].z, q[i].w};
            }
        }
    }
}

// Workgroup L of a launch over the (row group, K slice) items of `a`.
template <int F, int KS, int NT, int MT>
__device__ __forceinline__ void kq_body(const KqArgs &a, int L) {
    using G = KqGeom<F>;
    constexpr bool Q6 = F == kFQ6K;
    constexpr bool SUMS = F == kFQ4K;            // the min term needs sub-block sums of x
    constexpr int SBS = KS / 256;                // super-blocks per slice
    constexpr int RS = KS + 8;                   // x row stride (halves)
    constexpr int XSS = KS / 32 + 8;             // sub-block-sum row stride (halves)
    extern __shared__ uint8_t smem[];
    // x as hi and lo fp16 rows; Q4_K: split sub-block sums.
    _Float16 *xh = reinterpret_cast<_Float16 *>(smem);
    _Float16 *xl = xh + 32 * RS;
    _Float16 *sh = xl + 32 * RS;
    _Float16 *sl = sh + (SUMS ? 32 * XSS : 0);
    uint8_t *stage_base = reinterpret_cast<uint8_t *>(sl + (SUMS ? 32 * XSS : 0));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;
    const int nl = lane & 31;
    uint8_t *st = stage_base + wave * (32 * G::STR);
    // XCD-aware order: workgroup L runs on XCD L % 8. A 512-element unit of
    // these formats is not a whole number of 128-byte lines, so neighbouring
    // K slices of a row read the line between them, and on two XCDs it came
    // from HBM twice (1.3-1.5x the weight bytes measured). When the row-group
    // count is a multiple of 8, slice-major order already keeps a row group
    // on one XCD; otherwise XCD x takes the contiguous run [x * per,
    // (x + 1) * per) of the (row group, slice) items in row-major order.
    const int total = a.groups * a.slices;
    int rgrp, slice;
    if ((a.groups & 7) == 0) {
        if (L >= total) return;
        slice = L / a.groups;
        rgrp = L - slice * a.groups;
    } else {
        const int per = (total + 7) / 8;
        const int item = (L & 7) * per + (L >> 3);
        if (item >= total) return;
        rgrp = item / a.slices;
        slice = item - rgrp * a.slices;
    }
    const int ks0 = slice * KS;

    // Activation slice -> split fp16 rows (rows >= M zero); Q4_K also the
    // split sums of each 32-element sub-block.
    constexpr int XF4 = 32 * (KS / 4) / kThreads;
    static_assert(32 * (KS / 4) % kThreads == 0 && (KS / 4) % 8 == 0, "x slice split");
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
        const int i = tid + kThreads * j;
        const int m = i / (KS / 4), c = i % (KS / 4);
        f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (m < a.M) v = *reinterpret_cast<const f32x4 *>(a.x + static_cast<size_t>(m) * a.K + ks0 + 4 * c);
        const uint32_t p0 = pack_half2(v.x, v.y), p1 = pack_half2(v.z, v.w);
        const half2v h0 = __builtin_bit_cast(half2v, p0), h1 = __builtin_bit_cast(half2v, p1);
        const uint32_t q0 = pack_half2(v.x - static_cast<float>(h0.x), v.y - static_cast<float>(h0.y));
        const uint32_t q1 = pack_half2(v.z - static_cast<float>(h1.x), v.w - static_cast<float>(h1.y));
        *reinterpret_cast<uint2 *>(xh + m * RS + 4 * c) = make_uint2(p0, p1);
        *reinterpret_cast<uint2 *>(xl + m * RS + 4 * c) = make_uint2(q0, q1);
        if constexpr (SUMS) {
            float t = (v.x + v.y) + (v.z + v.w);
            // 8 consecutive float4s (lanes c%8 = 0..7 of one row) form a sub-block.
            t += __shfl_xor(t, 1);
            t += __shfl_xor(t, 2);
            t += __shfl_xor(t, 4);
            if ((c & 7) == 0) {
                const _Float16 th = static_cast<_Float16>(t);
                sh[m * XSS + (c >> 3)] = th;
                sl[m * XSS + (c >> 3)] = static_cast<_Float16>(t - static_cast<float>(th));
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    constexpr int U = NT * SBS;
    constexpr int W = 2;
    KqTile tr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) tr[t] = kq_tile(a, rgrp * (kRowsPerWg * NT) + t * kRowsPerWg + wave * 32);
    u32x4 qc[U][G::LOADS];
#pragma unroll
    for (int u = 0; u < W && u < U; ++u) issue_unit<F>(qc[u], a, tr[u / SBS], ks0 / 256 + u % SBS, lane);
    __syncthreads();

    f32x16 acc = {};
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (u + W < U) issue_unit<F>(qc[u + W], a, tr[(u + W) / SBS], ks0 / 256 + (u + W) % SBS, lane);
        const int t = u / SBS, sbl = u % SBS;
        if (sbl == 0) acc = f32x16{};
        stage_unit<F>(st, qc[u], lane);
        const uint8_t *row = st + nl * G::STR;   // this lane's weight row
        const _Float16 *xrh = xh + nl * RS + 256 * sbl + 8 * h;
        const _Float16 *xrl = xl + nl * RS + 256 * sbl + 8 * h;
        f32x16 cq = {};
        float d = 1.0f;
        if constexpr (F == kFQ40 || F == kFQ80) {
            // Eight 32-element blocks: fp16 d, then 16 (Q4_0) or 32 (Q8_0) code bytes.
            constexpr int BLK = F == kFQ40 ? 18 : 34;
            static_assert(MT == 8, "Q4_0 / Q8_0 passes hold at most 8 tokens");
            constexpr int RU = 4;                  // accumulators of rows m < 8
            const uint32_t one = int_half2(1, 1.0f);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const float db = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(row + BLK * b));
                const int e0 = 256 * sbl + 32 * b + 8 * h;
                f32x16 cb = {};
                if constexpr (F == kFQ40) {
                    uint32_t w0, w1;
                    lds_bytes8(row + BLK * b + 2 + 8 * h, (BLK * b + 2) & 3, w0, w1);
                    const half8 blo = fma_frag(w0 & 0x0f0f0f0fu, w1 & 0x0f0f0f0fu, one, int_half2(-1032, 1.0f));
                    const half8 bhi = fma_frag(w0 & 0xf0f0f0f0u, w1 & 0xf0f0f0f0u, int_half2(1, 0.0625f),
                                               int_half2(-72, 1.0f));
                    cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xh + nl * RS + e0), blo, cb, 0, 0, 0);
                    cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xl + nl * RS + e0), blo, cb, 0, 0, 0);
                    cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xh + nl * RS + e0 + 16), bhi, cb, 0, 0, 0);
                    cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xl + nl * RS + e0 + 16), bhi, cb, 0, 0, 0);
                } else {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        uint32_t w0, w1;
                        lds_bytes8(row + BLK * b + 2 + 16 * j + 8 * h, (BLK * b + 2) & 3, w0, w1);
                        const half8 bq = fma_frag(w0 ^ 0x80808080u, w1 ^ 0x80808080u, one, int_half2(-1152, 1.0f));
                        cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xh + nl * RS + e0 + 16 * j), bq, cb, 0, 0, 0);
                        cb = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xl + nl * RS + e0 + 16 * j), bq, cb, 0, 0, 0);
                    }
                }
#pragma unroll
                for (int r = 0; r < RU; ++r) cq[r] = fmaf(db, cb[r], cq[r]);
            }
        } else if constexpr (!Q6) {
            const u32x2v h01 = *reinterpret_cast<const u32x2v *>(row);
            const u32x2v h23 = *reinterpret_cast<const u32x2v *>(row + 8);
            const uint32_t sw0 = h01.y, sw1 = h23.x, sw2 = h23.y;   // the 12 scale/min bytes
            d = f16_bits_to_f32(h01.x & 0xffffu);
            float dmin = f16_bits_to_f32(h01.x >> 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                // Sub-blocks 2c (low nibbles) and 2c+1 (high nibbles) of qs[32c .. 32c+32).
                uint32_t sc0, sc1;
                if (c < 2) {
                    sc0 = __builtin_amdgcn_ubfe(sw0, 16 * c, 6);
                    sc1 = __builtin_amdgcn_ubfe(sw0, 16 * c + 8, 6);
                } else {
                    sc0 = __builtin_amdgcn_ubfe(sw2, 16 * (c - 2), 4) | (__builtin_amdgcn_ubfe(sw0, 16 * (c - 2) + 6, 2) << 4);
                    sc1 = __builtin_amdgcn_ubfe(sw2, 16 * (c - 2) + 8, 4) |
                          (__builtin_amdgcn_ubfe(sw0, 16 * (c - 2) + 14, 2) << 4);
                }
                const uint32_t mul_lo = int_half2(static_cast<int>(sc0), 1.0f);
                const uint32_t add_lo = int_half2(static_cast<int>(sc0), -1024.0f);
                const uint32_t mul_hi = int_half2(static_cast<int>(sc1), 0.0625f);
                const uint32_t add_hi = int_half2(static_cast<int>(sc1), -64.0f);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const u32x2v b = *reinterpret_cast<const u32x2v *>(row + 16 + 32 * c + 16 * j + 8 * h);
                    const half8 blo = fma_frag(b.x & 0x0f0f0f0fu, b.y & 0x0f0f0f0fu, mul_lo, add_lo);
                    const half8 bhi = fma_frag(b.x & 0xf0f0f0f0u, b.y & 0xf0f0f0f0u, mul_hi, add_hi);
                    const int e_lo = 64 * c + 16 * j, e_hi = e_lo + 32;
                    cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xrh + e_lo), blo, cq, 0, 0, 0);
                    cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xrl + e_lo), blo, cq, 0, 0, 0);
                    cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xrh + e_hi), bhi, cq, 0, 0, 0);
                    cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xrl + e_hi), bhi, cq, 0, 0, 0);
                }
            }
            // A block whose min codes are all zero has no min term, whatever
            // dmin holds (GRT/GgufQ4RawDot.java:38-148; a NaN dmin adds nothing).
            if (sw1 == 0 && (sw2 & 0xf0f0f0f0u) == 0) dmin = 0.0f;
            // Min term: A = split sub-block sums of this super-block (lane half
            // 0; half 1 supplies zeros), B = min codes.
            half8 amh = {}, aml = {}, bm = {};
            if (h == 0) {
                amh = *reinterpret_cast<const half8 *>(sh + nl * XSS + 8 * sbl);
                aml = *reinterpret_cast<const half8 *>(sl + nl * XSS + 8 * sbl);
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    bm[s] = static_cast<_Float16>(static_cast<float>(__builtin_amdgcn_ubfe(sw1, 8 * s, 6)));
                    bm[s + 4] = static_cast<_Float16>(static_cast<float>(
                        __builtin_amdgcn_ubfe(sw2, 8 * s + 4, 4) | (__builtin_amdgcn_ubfe(sw1, 8 * s + 6, 2) << 4)));
                }
            }
            f32x16 cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(amh, bm, f32x16{}, 0, 0, 0);
            cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(aml, bm, cm, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = fmaf(-dmin, cm[r], acc[r]);
        } else {
            d = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(row + 208));
            const u32x2v s01 = *reinterpret_cast<const u32x2v *>(row + 192);
            const u32x2v s23 = *reinterpret_cast<const u32x2v *>(row + 200);
            const uint32_t scw[4] = {s01.x, s01.y, s23.x, s23.y};
#pragma unroll
            for (int H = 0; H < 2; ++H) {
#pragma unroll
                for (int l16 = 0; l16 < 2; ++l16) {
                    // Elements 128H + 32q + 16*l16 + 8h + e for quadrants q = 0..3:
                    // ql bytes 64H + 32(q&1) + l, nibble q>>1; qh byte 32H + l, bits 2q.
                    const int l = 16 * l16 + 8 * h;
                    const u32x2v qa = *reinterpret_cast<const u32x2v *>(row + 64 * H + l);
                    const u32x2v qb = *reinterpret_cast<const u32x2v *>(row + 64 * H + 32 + l);
                    const u32x2v qh = *reinterpret_cast<const u32x2v *>(row + 128 + 32 * H + l);
                    uint32_t six[4][2];
#pragma unroll
                    for (int w = 0; w < 2; ++w) {
                        const uint32_t A = w ? qa.y : qa.x, B = w ? qb.y : qb.x, Q = w ? qh.y : qh.x;
                        six[0][w] = (A & 0x0f0f0f0fu) | ((Q << 4) & 0x30303030u);
                        six[1][w] = (B & 0x0f0f0f0fu) | ((Q << 2) & 0x30303030u);
                        six[2][w] = ((A >> 4) & 0x0f0f0f0fu) | (Q & 0x30303030u);
                        six[3][w] = ((B >> 4) & 0x0f0f0f0fu) | ((Q >> 2) & 0x30303030u);
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int g = 8 * H + 2 * q + l16;   // scale group of these 16 elements
                        const int sv = static_cast<int8_t>((scw[g >> 2] >> (8 * (g & 3))) & 0xffu);
                        const int sl = sv & 15;
                        half8 blo, bhi, bsum;
                        q6_frags(six[q][0], six[q][1], int_half2(sl, 1.0f), int_half2(sv - sl, 1.0f), blo, bhi, bsum);
                        const half8 ah = *reinterpret_cast<const half8 *>(xrh + 16 * g);
                        cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, blo, cq, 0, 0, 0);
                        cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bhi, cq, 0, 0, 0);
                        cq = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(xrl + 16 * g), bsum, cq, 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = fmaf(d, cq[r], acc[r]);
        __builtin_amdgcn_sched_barrier(0);
        if (sbl == SBS - 1) {
            const int n = tr[t].local0 + nl;
            if (n < tr[t].n) {
                if (a.slices == 1) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = 8 * (r >> 2) + 4 * h + (r & 3);
                        if (m < a.M) {
                            float *yp = tr[t].y + static_cast<size_t>(m) * tr[t].n + n;
                            *yp = a.add ? *yp + acc[r] : acc[r];
                        }
                    }
                } else {
                    // This slice's partial tile; the slice sum adds the
                    // slices in order.
                    float *ps = a.part + static_cast<size_t>(slice) * a.M * a.ld + a.col0 +
                                rgrp * (kRowsPerWg * NT) + t * kRowsPerWg + wave * 32 + nl;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = 8 * (r >> 2) + 4 * h + (r & 3);
                        if (m < a.M) ps[static_cast<size_t>(m) * a.ld] = acc[r];
                    }
                }
            }
        }
    }
}

template <int F, int KS, int NT, int MT>
__global__ __launch_bounds__(kThreads) void kq_mm_kernel(KqArgs a) {
    kq_body<F, KS, NT, MT>(a, static_cast<int>(blockIdx.x));
}

// Two formats in one launch: workgroups [0, nb0) take a0's items, the rest
// a1's (nb0 is a multiple of 8, so both parts keep their XCD order). Q and K
// of one K-quant beside V of another fill the chip together instead of V's
// few workgroups running alone.
template <int F0, int F1, int KS, int MT>
__global__ __launch_bounds__(kThreads) void kq_mm_mix_kernel(KqArgs a0, KqArgs a1, int nb0) {
    const int L = static_cast<int>(blockIdx.x);
    if (L < nb0) kq_body<F0, KS, 1, MT>(a0, L);
    else kq_body<F1, KS, 1, MT>(a1, L - nb0);
}

template <int F, int KS, int NT, int MT>
void launch_kq(const KqArgs &args, hipStream_t s) {
    static bool lds_set = false;                 // the attribute is per kernel, per process
    const void *fn = reinterpret_cast<const void *>(kq_mm_kernel<F, KS, NT, MT>);
    const size_t lds = kq_lds_bytes<F, KS>();
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        lds_set = true;
    }
    KqArgs a = args;
    a.groups = (args.N + kRowsPerWg * NT - 1) / (kRowsPerWg * NT);
    a.slices = args.K / KS;
    const int total = a.groups * a.slices;
    const int grid = (a.groups & 7) == 0 ? total : 8 * ((total + 7) / 8);
    hipLaunchKernelGGL((kq_mm_kernel<F, KS, NT, MT>), dim3(grid), dim3(kThreads), lds, s, a);
}

template <int F, int MT>
void launch_kq_nt(const KqArgs &args, int ks, int nt, hipStream_t s) {
    constexpr bool kFour = F == kFQ4K || F == kFQ40;
    if (ks == 256) {
        launch_kq<F, 256, 1, MT>(args, s);
    } else if (nt == 4 && kFour) {
        if constexpr (kFour) launch_kq<F, 512, 4, MT>(args, s);
    } else if (nt >= 2) {
        launch_kq<F, 512, 2, MT>(args, s);
    } else {
        launch_kq<F, 512, 1, MT>(args, s);
    }
}

}  // namespace

bool kquant_mfma_type(int type) {
    return type == ALJABR_ROCM_TYPE_Q4_K || type == ALJABR_ROCM_TYPE_Q6_K || type == ALJABR_ROCM_TYPE_Q4_0 ||
           type == ALJABR_ROCM_TYPE_Q8_0;
}

int kquant_mfma_max_m(int type) {
    return type == ALJABR_ROCM_TYPE_Q4_0 || type == ALJABR_ROCM_TYPE_Q8_0 ? 8 : 32;
}

namespace {

// The launch arguments of up to three matrices of one type (all but the last
// with a multiple of 32 rows): 2 <= M <= kquant_mfma_max_m(type),
// K % 512 == 0, A and weights 16-byte aligned.
int kq_multi_args(const KqOut *outs, int nseg, const float *A, int K, int type, int M, KqArgs &args) {
    if (!kquant_mfma_type(type) || nseg < 1 || nseg > 3 || M < 2 || M > kquant_mfma_max_m(type) || K % 512 != 0 ||
        !aligned(A, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    args = KqArgs{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const KqOut &o = outs[i];
            if (o.n <= 0 || !aligned(o.w, 16) || (i < nseg - 1 && o.n % 32 != 0)) return ALJABR_ROCM_ERR_UNSUPPORTED;
            end += o.n;
            if (end > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.y[i] = o.y;
            args.w[i] = o.w;
            args.end[i] = static_cast<int>(end);
        } else {
            args.end[i] = 0x7fffffff;
        }
    }
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    args.ld = args.N;
    return ALJABR_ROCM_OK;
}

// K slice of a launch: 512 elements, or 256 when 512-element slices would
// leave at least half the CUs without a workgroup (twice the workgroups,
// each with half the slice).
int kq_slice(int N, int K) {
    const int wgs_n = (N + kRowsPerWg - 1) / kRowsPerWg;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    return 2LL * wgs_n * (K / 512) <= cus ? 256 : 512;
}

void kq_launch(const KqArgs &args, int type, int ks, hipStream_t s) {
    const int wgs_n = (args.N + kRowsPerWg - 1) / kRowsPerWg;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    // Row tiles per wave: 1, 2 when one leaves more workgroups than CUs, 4
    // when two still do (every workgroup resident at once instead of a ragged second batch;
    // Q4_K and Q4_0 only: Q6_K's and Q8_0's four-tile kernels reach the
    // register limit).
    const long long units = static_cast<long long>(wgs_n) * (args.K / 512);
    const bool four_ok = type == ALJABR_ROCM_TYPE_Q4_K || type == ALJABR_ROCM_TYPE_Q4_0;
    const int nt = units <= cus ? 1 : (units + 1) / 2 <= cus || !four_ok ? 2 : 4;
    switch (type) {
    case ALJABR_ROCM_TYPE_Q4_K: launch_kq_nt<kFQ4K, 32>(args, ks, nt, s); break;
    case ALJABR_ROCM_TYPE_Q6_K: launch_kq_nt<kFQ6K, 32>(args, ks, nt, s); break;
    case ALJABR_ROCM_TYPE_Q4_0: launch_kq_nt<kFQ40, 8>(args, ks, nt, s); break;
    default: launch_kq_nt<kFQ80, 8>(args, ks, nt, s); break;
    }
}

}  // namespace

// With `tail` (K >= 1024, not accumulating) the slice sums go to the tail
// kernel instead of the outputs.
int enqueue_kquant_mfma_multi(const KqOut *outs, int nseg, const float *A, int K, int type, int M, bool accumulate,
                              float *part, size_t part_floats, const SliceTail *tail, const uint16_t *xpacked) {
    KqArgs args;
    const int rc = kq_multi_args(outs, nseg, A, K, type, M, args);
    if (rc != ALJABR_ROCM_OK) return rc;
    if (tail && (accumulate || K < 1024)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (type == ALJABR_ROCM_TYPE_Q4_0 || type == ALJABR_ROCM_TYPE_Q8_0) {
        // The activation-stationary kernel where the shape fits it.
        RowsOut o[3];
        for (int i = 0; i < nseg; ++i) o[i] = RowsOut{outs[i].y, outs[i].w, nullptr, outs[i].n};
        const int r = gguf_gemm_pass(o, nseg, A, K, type, M, accumulate, part, part_floats, tail);
        if (r != ALJABR_ROCM_ERR_UNSUPPORTED) return r;
    } else if (type == ALJABR_ROCM_TYPE_Q4_K) {
        RowsOut o[3];
        for (int i = 0; i < nseg; ++i) o[i] = RowsOut{outs[i].y, outs[i].w, nullptr, outs[i].n};
        const int r = q4k_gemm_pass(o, nseg, A, K, M, accumulate, part, part_floats, tail, xpacked);
        if (r != ALJABR_ROCM_ERR_UNSUPPORTED) return r;
    }
    hipStream_t s = current_stream();
    const int ks = kq_slice(args.N, K);
    const int slices = K / ks;
    args.add = slices == 1 && accumulate;
    if (slices > 1) {
        const size_t need = static_cast<size_t>(slices) * M * args.N;
        args.part = part && need <= part_floats
                        ? part
                        : static_cast<float *>(stream_scratch(need * sizeof(float), kScratchPartials));
        if (!args.part) return ALJABR_ROCM_ERR_BUFFER;
    }
    kq_launch(args, type, ks, s);
    if (tail) return enqueue_slice_tail(*tail, args.part, slices, M, args.N);
    if (slices > 1) {
        float *ys[3] = {args.y[0], args.y[1], args.y[2]};
        return enqueue_slice_sum(ys, args.end, nseg, M, args.N, args.part, slices, accumulate);
    }
    return ALJABR_ROCM_OK;
}

int enqueue_kquant_mfma_parts(const KqOut *outs, int nseg, const float *A, int K, int type, int M, float *part,
                              size_t part_floats, int ld, int col0) {
    KqArgs args;
    const int rc = kq_multi_args(outs, nseg, A, K, type, M, args);
    if (rc != ALJABR_ROCM_OK) return rc;
    const int slices = K / 512;
    if (slices < 2 || !part || col0 < 0 || col0 % 32 != 0 || static_cast<long long>(col0) + args.N > ld ||
        static_cast<size_t>(slices) * M * ld > part_floats)
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.part = part;
    args.ld = ld;
    args.col0 = col0;
    kq_launch(args, type, 512, current_stream());
    return ALJABR_ROCM_OK;
}

int enqueue_kquant_mfma_parts2(const KqOut *outs0, int nseg0, int type0, const KqOut *outs1, int nseg1, int type1,
                               const float *A, int K, int M, float *part, size_t part_floats) {
    if (type0 != ALJABR_ROCM_TYPE_Q4_K || type1 != ALJABR_ROCM_TYPE_Q6_K) return ALJABR_ROCM_ERR_UNSUPPORTED;
    KqArgs a0, a1;
    int rc = kq_multi_args(outs0, nseg0, A, K, type0, M, a0);
    if (rc != ALJABR_ROCM_OK) return rc;
    rc = kq_multi_args(outs1, nseg1, A, K, type1, M, a1);
    if (rc != ALJABR_ROCM_OK) return rc;
    const int slices = K / 512;
    const long long ld = static_cast<long long>(a0.N) + a1.N;
    if (slices < 2 || !part || a0.N % 32 != 0 || ld > 0x7fff0000LL ||
        static_cast<size_t>(slices) * M * static_cast<size_t>(ld) > part_floats)
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    a0.part = a1.part = part;
    a0.ld = a1.ld = static_cast<int>(ld);
    a0.col0 = 0;
    a1.col0 = a0.N;
    KqArgs *as[2] = {&a0, &a1};
    int grid[2];
    for (int i = 0; i < 2; ++i) {
        KqArgs &a = *as[i];
        a.groups = (a.N + kRowsPerWg - 1) / kRowsPerWg;
        a.slices = slices;
        const int total = a.groups * a.slices;
        grid[i] = (a.groups & 7) == 0 ? total : 8 * ((total + 7) / 8);
    }
    // One tile per wave (the single-format launch's choice while its items
    // fit the CUs), both parts resident at once.
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    if (grid[0] + grid[1] > cus) return ALJABR_ROCM_ERR_UNSUPPORTED;
    constexpr int F0 = kFQ4K, F1 = kFQ6K;
    const void *fn = reinterpret_cast<const void *>(kq_mm_mix_kernel<F0, F1, 512, 32>);
    const size_t lds = std::max(kq_lds_bytes<F0, 512>(), kq_lds_bytes<F1, 512>());
    static bool lds_set = false;
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        lds_set = true;
    }
    hipLaunchKernelGGL((kq_mm_mix_kernel<F0, F1, 512, 32>), dim3(grid[0] + grid[1]), dim3(kThreads), lds,
                       current_stream(), a0, a1, grid[0]);
    return ALJABR_ROCM_OK;
}

int enqueue_kquant_mfma(float *C, const float *A, const uint8_t *W, int K, int N, int type, int M, float *part,
                        size_t part_floats) {
    const KqOut o{C, W, N};
    return enqueue_kquant_mfma_multi(&o, 1, A, K, type, M, false, part, part_floats);
}

size_t kquant_mfma_scratch_floats(int M, int N, int K) {
    if (M < 2 || N < 1 || K % 512 != 0) return 0;
    const int slices = K / kq_slice(N, K);
    const size_t kq = slices > 1 ? static_cast<size_t>(slices) * M * N : 0;
    // The Q4_K register-resident kernel's partials and fp16 A image.
    const size_t q4k = q4k_gemm_scratch_floats(M, N, K);
    return kq > q4k ? kq : q4k;
}

}  // namespace aljabr
