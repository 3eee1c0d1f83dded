// matvec_rows.hip - batch-1 matvec for NF4, Q4_0 and Q8_0 rows, K split
// across the waves of a workgroup, T rows per wave pipelined in straight-line
// code.
//
// Formats (reference layouts):
//   NF4  codes u8[N*K/2], byte j = (code[2j] << 4) | code[2j+1], absmax fp32
//        per 2^k >= 32 elements of the flat [N,K] index
//        (STC/DequantizationKernel.java:84-102);
//   Q4_0 18-byte blocks {f16 d; u8 qs[16]}, qs[j] low nibble -> element j,
//        high nibble -> element j+16, value (q-8)*d
//        (GRT/GgufBlockDequantizer.java:33-37,403-416);
//   Q8_0 34-byte blocks {f16 d; i8 qs[32]} (GRT/GgufBlockDequantizer.java:231-265);
//   Q4_K / Q6_K 144- / 210-byte super-blocks of 256 weights, 8 lanes per
//        super-block (layouts and lane split in kquant.hpp).
//
// Decoding is the bottleneck once the weights stream at HBM speed, so every
// choice below cuts VALU instructions per weight:
//   * 4-bit formats decode a whole code BYTE (two weights) with one LDS read of
//     a float2 from a 256-entry pair table. The table is replicated 32 times,
//     entry e of replica r at byte address e*256 + r*8, so lane l reads replica
//     l%32 and a wave's reads never conflict; and the address is one v_perm_b32
//     (code byte into bits 8-15, the lane's r*8 into bits 0-7). Per weight:
//     half a v_perm, half an LDS read, one FMA.
//   * Q8_0 converts each signed code byte with one sign-extending byte
//     convert (v_cvt_f32_i32 with an SDWA byte select): one convert and one
//     FMA per weight.
//   * Q4_K takes the pair table of raw nibbles; Q6_K masks the nibbles and
//     merges its two high bits four bytes at a time and converts with
//     v_cvt_f32_ubyte. The per-sub-block scale is applied to the lane's two
//     partial dots, the Q4_K min and the Q6_K -32 offset through the lane's
//     activation sums.
//   * Activations are staged once per workgroup with coalesced loads through
//     a swizzled LDS window (conflict-free), then live in registers: lane l
//     owns the 32 weights [32l, 32l+32) of its wave's 2048-element K chunk.
//   * Each wave streams T contiguous rows, unrolled with the loads of row
//     t+PF issued before row t is computed (the compiler drains all loads at
//     a loop back-edge), and the T row sums are reduced across the wave by
//     one butterfly.
//
// Workgroup = W (8 or 16) waves: G = W/S row groups of S = K/2048 K-chunk
// waves (waves beyond S*G only help with set-up). Q4_0/Q8_0 rows are read per lane PAIR:
// lanes 2m and 2m+1 own blocks 2m, 2m+1, 36 (Q4_0) or 68 (Q8_0) bytes that
// start 4-byte aligned when K % 64 == 0, so each lane loads dwords that lie
// inside its pair and realigns its block with one v_perm per word.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"
#include "kquant.hpp"

namespace aljabr {
namespace {

constexpr int kChunk = 2048;
constexpr int kFmtNF4 = 0, kFmtQ4 = 1, kFmtQ8 = 2, kFmtQ4K = 3, kFmtQ6K = 4;
constexpr bool kquant_fmt(int f) { return f == kFmtQ4K || f == kFmtQ6K; }
constexpr bool pair_table_fmt(int f) { return f == kFmtNF4 || f == kFmtQ4 || f == kFmtQ4K; }
// Dynamic LDS: [0, kMainBytes) the pair table, [kMainBytes, 2 kMainBytes)
// the activation windows (S windows of 8 KiB), then the wave partials and the
// RMSNorm chunk sums. The table and the windows do not overlap, so the table
// is built while the activations are still in flight and one barrier covers
// both. The kernel declares no static LDS, so the table starts at address 0
// and a lookup address is the v_perm result itself (a nonzero base costs one
// v_add per lookup: the compiler cannot fold it into the ds_read offset
// because the permuted address is not known to be non-negative).
constexpr int kMainBytes = 256 * 256;   // 256 pair entries x 32 replicas x float2
constexpr int kLdsBytes = 2 * kMainBytes;

typedef unsigned int u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4a4 load_stream16_a4(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4a4 *>(p));
}
__device__ __forceinline__ uint32_t load_stream4(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}

// Per-lane raw data of one row.
template <int FMT> struct RowWords;
template <> struct RowWords<kFmtNF4> { u32x4 q; float s; };
template <> struct RowWords<kFmtQ4> { u32x4a4 a; uint32_t b; };
template <> struct RowWords<kFmtQ8> { u32x4a4 a, b; uint32_t c; };
template <> struct RowWords<kFmtQ4K> : Q4KWords {};
template <> struct RowWords<kFmtQ6K> : Q6KWords {};

// Float4 f of the wave's 2048-element activation chunk that fills xv[4i..4i+4)
// of `lane`: 32 consecutive elements, or for the K-quants the lane's 16 low
// then 16 high elements of its super-block.
template <int FMT>
__device__ __forceinline__ int x_f4(int lane, int i) {
    if constexpr (FMT == kFmtQ4K || FMT == kFmtQ6K) {
        const int j = lane & 7;
        const int e = 256 * (lane >> 3) + (FMT == kFmtQ4K ? q4k_lo_elem(j) : q6k_lo_elem(j)) +
                      (i >= 4 ? (FMT == kFmtQ4K ? kQ4KHigh : kQ6KHigh) : 0);
        return (e >> 2) + (i & 3);
    } else {
        return lane * 8 + i;
    }
}

// A launch covers up to three weight matrices of the same K stacked as one
// row space (the decode step's Q/K/V or gate/up share one launch and one
// activation staging); segment s owns rows [seg[s-1].end, seg[s].end), or,
// for the SwiGLU epilogue, stacked row 2i is row i of segment 0 and 2i+1 row
// i of segment 1 (so a gate row and its up row meet in one wave).
struct RowsSeg {
    const uint8_t *w;
    const float *absmax;   // NF4 only
    float *y;
    int end;               // one past the segment's last row in the stacked row space
};

// Prologue applied to the activations while they are staged, and epilogue of
// the row sums.
constexpr int kXPlain = 0;     // x
constexpr int kXNorm = 1;      // RMSNorm: (x * 1/sqrt(mean(x^2) + eps)) * norm_w
constexpr int kEStore = 0;     // y = v
constexpr int kEStore3 = 4;    // y = v, three stacked segments (segment 2's pointers read from the struct)
constexpr int kEAdd = 1;       // y += v (residual)
constexpr int kESwiGLU = 2;    // interleaved gate/up pairs: y = silu(gate) * up
constexpr int kERopeKV = 3;    // Q/K/V pairs: RoPE on q (stored) and k, k and v appended to the fp16 caches

struct RowsArgs {
    RowsSeg seg[3];
    const float *x;
    const float *norm_w;   // kXNorm
    float eps;
    // kERopeKV (one sequence): position, this layer's caches [n_kv][cap][D],
    // D = 2^hd_shift.
    const int *pos;
    uint16_t *kc, *vc;
    int cap, hd_shift;
    float rope_base;
    const float2 *rope_cs;   // [cap][D/2] cos/sin table, or null
    int N, K, bs_shift, S, G;
    int gelu;                // kESwiGLU: the tanh GELU of the Metal FFN instead of SiLU
};

// The arguments a wave needs before its first weight load: segments 0 and 1
// (pointers and ends), the activations and the shape. rows_kernel takes them
// as its leading scalar arguments, which the build preloads into SGPRs at wave
// launch (14 dwords, the hardware limit); read from the argument struct they
// cost two dependent scalar-memory round trips (the shape, then the
// pointers), ~0.7 us before the first weight request under a full HBM queue.
// K = S * 2048 on this path, so the shape packs into one word:
// S | G << 4 | bs_shift << 9 | hd_shift << 14.
struct RowsHot {
    const float *x;
    const uint8_t *w0, *w1, *w2;
    const float *s0, *s1, *s2;   // NF4 absmax of segments 0, 1 and 2
    int N, end0, end1;
    int S, G, K, bs_shift, hd_shift;
};

__host__ __device__ inline int rows_shape_word(const RowsArgs &a) {
    return a.S | (a.G << 4) | (a.bs_shift << 9) | (a.hd_shift << 14);
}

__device__ __forceinline__ RowsHot rows_hot(const float *x, const uint8_t *w0, const float *s0, const uint8_t *w1,
                                            const float *s1, int N, int end0, int end1, int shape) {
    RowsHot h;
    h.x = x;
    h.w0 = w0;
    h.w1 = w1;
    h.s0 = s0;
    h.s1 = s1;
    h.N = N;
    h.end0 = end0;
    h.end1 = end1;
    h.S = shape & 15;
    h.G = (shape >> 4) & 31;
    h.K = h.S * kChunk;
    h.bs_shift = (shape >> 9) & 31;
    h.hd_shift = (shape >> 14) & 15;
    h.w2 = w0;               // set by with_seg2 for three-segment launches
    h.s2 = s0;
    return h;
}

// Segment 2's pointers live only in the argument struct, so only the
// epilogues of three-segment launches (kEStore3, kERopeKV) read them: every
// other launch starts its loads without waiting for the struct.
template <int EPI>
__device__ __forceinline__ void with_seg2(RowsHot &h, const RowsArgs &a) {
    if constexpr (EPI == kEStore3 || EPI == kERopeKV) {
        h.w2 = a.seg[2].w;
        h.s2 = a.seg[2].absmax;
    }
}

__device__ __forceinline__ RowsHot rows_hot(const RowsArgs &a) {
    RowsHot h = rows_hot(a.x, a.seg[0].w, a.seg[0].absmax, a.seg[1].w, a.seg[1].absmax, a.N, a.seg[0].end,
                         a.seg[1].end, rows_shape_word(a));
    h.w2 = a.seg[2].w;
    h.s2 = a.seg[2].absmax;
    return h;
}

// Segment of stacked row r and its row within the segment. The row map
// follows from the epilogue at compile time (per-row runtime tests cost the
// plain kernel over a microsecond): kESwiGLU interleaves two segments,
// kERopeKV pairs the rows of each q and k head. Segments are picked with the
// two comparisons directly (scalar selects).
struct RowRef {
    bool s1, s2;           // segment 1 or 2 (neither: segment 0)
    int local;
};

template <int EPI, int T>
__device__ __forceinline__ RowRef row_ref(const RowsHot &h, int r) {
    RowRef f;
    if constexpr (EPI == kESwiGLU) {
        // A wave's T rows are T/2 consecutive gate rows, then the same T/2 up
        // rows: both matrices are read as contiguous runs.
        const int blk = r / T, t = r - blk * T;
        f.s1 = t >= T / 2;
        f.s2 = false;
        f.local = blk * (T / 2) + (f.s1 ? t - T / 2 : t);
    } else {
        f.s1 = r >= h.end0;
        f.s2 = r >= h.end1;
        f.local = r - (f.s2 ? h.end1 : f.s1 ? h.end0 : 0);
        if constexpr (EPI == kERopeKV) {
            if (!f.s2) {
                const int hd = 1 << h.hd_shift, q = f.local & (hd - 1);
                f.local = (f.local - q) + (q >> 1) + (q & 1) * (hd >> 1);
            }
        }
    }
    return f;
}

template <class T>
__device__ __forceinline__ T seg_pick(const RowRef &f, T a0, T a1, T a2) {
    return f.s2 ? a2 : f.s1 ? a1 : a0;
}

// Per-lane byte offsets of a row's loads (loop-invariant): the row's address
// is a wave-uniform base plus these, so every load takes the scalar-base form
// and no row spends vector instructions on addresses.
struct LaneOffsets {
    uint32_t w;       // weight bytes from the row's chunk start
    uint32_t s;       // NF4: absmax bytes from the row's chunk block
};

template <int FMT>
__device__ __forceinline__ LaneOffsets lane_offsets(int lane, int bs_shift) {
    LaneOffsets o{};
    if constexpr (FMT == kFmtNF4) {
        o.w = static_cast<uint32_t>(lane) * 16u;
        o.s = (static_cast<uint32_t>(lane * 32) >> bs_shift) * 4u;
    } else if constexpr (kquant_fmt(FMT)) {
        constexpr uint32_t BB = FMT == kFmtQ4K ? kQ4KBytes : kQ6KBytes;
        o.w = static_cast<uint32_t>(lane >> 3) * BB;
    } else {
        // Pair start (4-byte aligned) + 16 (Q4_0) or 32 (Q8_0) for the odd lane.
        constexpr uint32_t BB = FMT == kFmtQ4 ? 18 : 34;
        o.w = static_cast<uint32_t>(lane >> 1) * (2 * BB) + static_cast<uint32_t>(lane & 1) * (BB - 2);
    }
    return o;
}

template <int FMT, int EPI, int T>
__device__ __forceinline__ void load_row(RowWords<FMT> &d, const RowsHot &h, const RowsArgs &a, int row, int chunk,
                                         const LaneOffsets &o) {
    const RowRef f = row_ref<EPI, T>(h, row);
    const size_t local = static_cast<size_t>(f.local);
    const uint8_t *w = seg_pick(f, h.w0, h.w1, h.w2);
    if constexpr (FMT == kFmtNF4) {
        // bs divides K here (bs <= 2048 = the chunk), so the row's blocks
        // start at local * K / bs.
        const float *absmax = seg_pick(f, h.s0, h.s1, h.s2);
        const uint8_t *rw = w + local * (static_cast<size_t>(h.K) >> 1) + static_cast<size_t>(chunk) * (kChunk / 2);
        const uint8_t *rs = reinterpret_cast<const uint8_t *>(
            absmax + ((local * static_cast<size_t>(h.K) + static_cast<size_t>(chunk) * kChunk) >> h.bs_shift));
        d.q = load_stream16(rw + o.w);
        d.s = *reinterpret_cast<const float *>(rs + o.s);
    } else if constexpr (kquant_fmt(FMT)) {
        constexpr int BB = FMT == kFmtQ4K ? kQ4KBytes : kQ6KBytes;
        const uint8_t *rw = w + local * (static_cast<size_t>(h.K >> 8) * BB) + static_cast<size_t>(chunk) * (8 * BB);
        const int j = __lane_id() & 7;
        if constexpr (FMT == kFmtQ4K) load_q4k(d, rw + o.w, j);
        else load_q6k(d, rw + o.w, j);
    } else {
        constexpr int BB = FMT == kFmtQ4 ? 18 : 34;
        const uint8_t *rw = w + local * (static_cast<size_t>(h.K >> 5) * BB) + static_cast<size_t>(chunk) * (64 * BB);
        const uint8_t *p = rw + o.w;
        if constexpr (FMT == kFmtQ4) {
            d.a = load_stream16_a4(p);
            d.b = load_stream4(p + 16);
        } else {
            d.a = load_stream16_a4(p);
            d.b = load_stream16_a4(p + 16);
            d.c = load_stream4(p + 32);
        }
    }
}

// LDS address of the pair-table entry for byte BYTE of `w`, replica in `cl`.
template <int BYTE>
__device__ __forceinline__ uint32_t pair_addr(uint32_t w, uint32_t cl) {
    return __builtin_amdgcn_perm(w, cl, 0x0C0C0000u | ((4u + BYTE) << 8));
}

// The table sits at LDS address 0 (kMainBytes), so the byte address is the
// LDS pointer itself; `tbl` is unused by the load.
__device__ __forceinline__ float2 pair_at(const char *, uint32_t addr) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef const f32x2 __attribute__((address_space(3))) lds_f32x2;
    const f32x2 v = *(lds_f32x2 *)(static_cast<uintptr_t>(addr));
    return make_float2(v.x, v.y);
}

// sum over the lane's 32 weights of w*x, before the row/block scale.
template <int FMT>
__device__ __forceinline__ float row_dot(const RowWords<FMT> &d, const float (&xv)[32], float xsum, float xsum2,
                                         uint32_t align_sel, uint32_t cl, const char *tbl, float &scale) {
    if constexpr (kquant_fmt(FMT)) {
        // xsum / xsum2: sums of the lane's low / high activations.
        const int j = __lane_id() & 7;
        float plo, phi;
        scale = 1.0f;
        if constexpr (FMT == kFmtQ4K) {
            // Pair table of raw nibbles: byte -> (low, high) as floats.
            const uint32_t wv[4] = {d.q.x, d.q.y, d.q.z, d.q.w};
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 e0 = pair_at(tbl, pair_addr<0>(wv[i], cl));
                const float2 e1 = pair_at(tbl, pair_addr<1>(wv[i], cl));
                const float2 e2 = pair_at(tbl, pair_addr<2>(wv[i], cl));
                const float2 e3 = pair_at(tbl, pair_addr<3>(wv[i], cl));
                p0 = fmaf(e0.x, xv[4 * i + 0], p0);
                p1 = fmaf(e0.y, xv[16 + 4 * i + 0], p1);
                p0 = fmaf(e1.x, xv[4 * i + 1], p0);
                p1 = fmaf(e1.y, xv[16 + 4 * i + 1], p1);
                p0 = fmaf(e2.x, xv[4 * i + 2], p0);
                p1 = fmaf(e2.y, xv[16 + 4 * i + 2], p1);
                p0 = fmaf(e3.x, xv[4 * i + 3], p0);
                p1 = fmaf(e3.y, xv[16 + 4 * i + 3], p1);
            }
            return k_combine<false>(q4k_scales(d.hdr, j), p0, p1, xsum, xsum2);
        } else {
            q6k_dots(d, j, xv, xv + 16, plo, phi);
            return k_combine<true>(q6k_scales(d, j), plo, phi, xsum, xsum2);
        }
    } else if constexpr (FMT == kFmtNF4) {
        const uint32_t wv[4] = {d.q.x, d.q.y, d.q.z, d.q.w};
        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 e0 = pair_at(tbl, pair_addr<0>(wv[i], cl));
            const float2 e1 = pair_at(tbl, pair_addr<1>(wv[i], cl));
            const float2 e2 = pair_at(tbl, pair_addr<2>(wv[i], cl));
            const float2 e3 = pair_at(tbl, pair_addr<3>(wv[i], cl));
            p0 = fmaf(e0.x, xv[8 * i + 0], p0);
            p1 = fmaf(e0.y, xv[8 * i + 1], p1);
            p0 = fmaf(e1.x, xv[8 * i + 2], p0);
            p1 = fmaf(e1.y, xv[8 * i + 3], p1);
            p0 = fmaf(e2.x, xv[8 * i + 4], p0);
            p1 = fmaf(e2.y, xv[8 * i + 5], p1);
            p0 = fmaf(e3.x, xv[8 * i + 6], p0);
            p1 = fmaf(e3.y, xv[8 * i + 7], p1);
        }
        scale = d.s;
        return p0 + p1;
    } else {
        // Realign: even lane's block starts 2 bytes into its first dword
        // (d = low half, codes from byte 2), odd lane's block starts 2 bytes
        // before it (d = high half of dword 0, codes from dword 1).
        constexpr int NW = FMT == kFmtQ4 ? 4 : 8;
        uint32_t dw[NW + 1];
        dw[0] = d.a.x; dw[1] = d.a.y; dw[2] = d.a.z; dw[3] = d.a.w;
        if constexpr (FMT == kFmtQ4) {
            dw[4] = d.b;
        } else {
            dw[4] = d.b.x; dw[5] = d.b.y; dw[6] = d.b.z; dw[7] = d.b.w; dw[8] = d.c;
        }
        // One v_perm per word with the lane's selector: bytes 2..5 of
        // (dw[i+1]:dw[i]) in even lanes, dw[i+1] in odd ones; the selector's
        // low half picks d the same way (bytes 0-1 or 2-3 of dw[0]).
        uint32_t qw[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) qw[i] = __builtin_amdgcn_perm(dw[i + 1], dw[i], align_sel);
        scale = f16_bits_to_f32(__builtin_amdgcn_perm(0u, dw[0], (align_sel & 0xffffu) - 0x0202u + 0x0c0c0000u));
        if constexpr (FMT == kFmtQ4) {
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 e0 = pair_at(tbl, pair_addr<0>(qw[i], cl));
                const float2 e1 = pair_at(tbl, pair_addr<1>(qw[i], cl));
                const float2 e2 = pair_at(tbl, pair_addr<2>(qw[i], cl));
                const float2 e3 = pair_at(tbl, pair_addr<3>(qw[i], cl));
                p0 = fmaf(e0.x, xv[4 * i + 0], p0);
                p1 = fmaf(e0.y, xv[16 + 4 * i + 0], p1);
                p0 = fmaf(e1.x, xv[4 * i + 1], p0);
                p1 = fmaf(e1.y, xv[16 + 4 * i + 1], p1);
                p0 = fmaf(e2.x, xv[4 * i + 2], p0);
                p1 = fmaf(e2.y, xv[16 + 4 * i + 2], p1);
                p0 = fmaf(e3.x, xv[4 * i + 3], p0);
                p1 = fmaf(e3.y, xv[16 + 4 * i + 3], p1);
            }
            return p0 + p1;
        } else {
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                // Signed codes converted directly: one sign-extending byte
                // convert per weight (an SDWA byte select).
                const uint32_t u = qw[i];
                p0 = fmaf(static_cast<float>(static_cast<int8_t>(u & 0xffu)), xv[4 * i + 0], p0);
                p1 = fmaf(static_cast<float>(static_cast<int8_t>((u >> 8) & 0xffu)), xv[4 * i + 1], p1);
                p0 = fmaf(static_cast<float>(static_cast<int8_t>((u >> 16) & 0xffu)), xv[4 * i + 2], p0);
                p1 = fmaf(static_cast<float>(static_cast<int8_t>(u >> 24)), xv[4 * i + 3], p1);
            }
            return p0 + p1;
        }
    }
}

// Pair table: slot i holds entry e = i/32 of replica i%32. NF4 bytes are (even code << 4) | odd code -> (level[hi],
// level[lo]); Q4_0 low nibble -> element j, high -> j+16 -> (lo-8, hi-8); Q4_K (lo, hi).
template <int FMT, int NT>
__device__ __forceinline__ void build_pair_table(float2 *tbl2, int tid) {
    static_assert(NT == 512 || NT == 1024, "table build assumes 512 or 1024 threads");
    constexpr float kNF4[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
    // Slot i = tid + NT*k: low nibble (i/32)%16 = (tid/32)%16, high nibble
    // i/512 = (NT/512)*k + tid/512.
    const int lo = (tid >> 5) & 15;
    const bool h1 = NT == 1024 && (tid >> 9);
    constexpr int zp = FMT == kFmtQ4 ? 8 : 0;   // Q4_0 zero point
    const float vlo = FMT == kFmtNF4 ? nf4_level_sel(lo) : static_cast<float>(lo - zp);
#pragma unroll
    for (int k = 0; k < 8192 / NT; ++k) {
        const int hi0 = (NT / 512) * k;
        const float vhi = FMT == kFmtNF4 ? (h1 ? kNF4[hi0 + 1] : kNF4[hi0])
                                         : static_cast<float>(hi0 - zp) + (h1 ? 1.0f : 0.0f);
        tbl2[tid + NT * k] = FMT == kFmtNF4 ? make_float2(vhi, vlo) : make_float2(vlo, vhi);
    }
}

__device__ __forceinline__ float silu_ref(float g) {
    // GGUFVectorOps.swiGLU's gate: g / (1 + Math.exp(-g)), exp in double.
    return g / (1.0f + static_cast<float>(exp(-static_cast<double>(g))));
}

// GELU(g) * u of the Metal FFN (MTLC/aljabr_metal_kernel_source.m:91-108):
// tanh GELU, 0 at or below -10 and g at or above 10; a non-finite product is 0.
__device__ __forceinline__ float geglu_metal(float g, float u) {
    float act;
    if (g <= -10.0f) act = 0.0f;
    else if (g >= 10.0f) act = g;
    else act = 0.5f * g * (1.0f + tanhf(0.79788456f * (g + 0.044715f * g * g * g)));
    const float y = act * u;
    return isfinite(y) ? y : 0.0f;
}


__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// P0 rows are requested before the set-up (table build, activation staging)
// and PF rows stay in flight afterwards: a deeper prologue keeps HBM busy
// while the activations arrive, a shallower steady state measured faster.
// One workgroup's rows: workgroup `blk` of a launch covering the stacked rows
// [row_base, row_end) in format FMT.
template <int FMT, int T, int PF, int W, int XOP, int EPI, int P0>
__device__ __forceinline__ void rows_body(RowsHot h, const RowsArgs &a, unsigned blk, int row_base, int row_end) {
    static_assert(T >= 1 && T <= 32 && PF >= 1 && P0 >= PF && (W == 8 || W == 16), "tile shape");
    constexpr int TP = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : T <= 16 ? 16 : 32;   // butterfly width
    extern __shared__ float4 smem[];    // see kMainBytes
    float(*part)[TP] = reinterpret_cast<float(*)[TP]>(reinterpret_cast<char *>(smem) + kLdsBytes);
    float *ssq = reinterpret_cast<float *>(reinterpret_cast<char *>(smem) + kLdsBytes) + W * TP;  // kXNorm
    f32x4 *xwin = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(smem) + kMainBytes);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave-uniform in a scalar register, so row and segment arithmetic is scalar.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = h.S;
    const int chunk = wave % S;
    const int grp = wave / S;
    float2 *tbl2 = reinterpret_cast<float2 *>(smem);

    if (grp >= h.G) {
        // Helper wave (when S does not divide W): takes part in the table
        // build and meets the same workgroup barriers, nothing else.
        if constexpr (pair_table_fmt(FMT)) build_pair_table<FMT, W * 64>(tbl2, tid);
        if constexpr (XOP == kXNorm) __syncthreads();        // 0: chunk sums of squares
        __syncthreads();                                     // 1: table built, x staged
        __syncthreads();                                     // 2: partials written
        return;
    }

    const bool stager = grp == 0;                // one wave per chunk stages x
    // Each wave streams the T contiguous rows row0 .. row0 + T-1 of the
    // stacked row space (measured a few percent faster on MI355X than
    // interleaving rows across the grid).
    const int row0 = row_base + static_cast<int>((blk * h.G + grp) * T);
    const int rstride = 1;
    const LaneOffsets lo = lane_offsets<FMT>(lane, h.bs_shift);
    with_seg2<EPI>(h, a);

    // Activations first (vmcnt retires in order: waiting for them then
    // leaves the weight loads in flight).
    const int xoff = chunk * kChunk;
    f32x4 xl[8], xm[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xl[j] = xm[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (stager) {
        const f32x4 *xw = reinterpret_cast<const f32x4 *>(h.x + xoff);
#pragma unroll
        for (int j = 0; j < 8; ++j) xl[j] = xw[64 * j + lane];
        if constexpr (XOP == kXNorm) {
            const f32x4 *mw = reinterpret_cast<const f32x4 *>(a.norm_w + xoff);
#pragma unroll
            for (int j = 0; j < 8; ++j) xm[j] = mw[64 * j + lane];
        }
    }
    RowWords<FMT> rw[T];
#pragma unroll
    for (int t = 0; t < P0 && t < T; ++t) load_row<FMT, EPI, T>(rw[t], h, a, min(row0 + t * rstride, row_end - 1), chunk, lo);
    // The table does not depend on the loads: build it while they fly.
    if constexpr (pair_table_fmt(FMT)) build_pair_table<FMT, W * 64>(tbl2, tid);

    if constexpr (XOP == kXNorm) {
        // RMSNorm over the whole row of K activations: chunk sums of squares
        // through LDS, then x * (1/sqrt(mean + eps)) * w in the same order as
        // the stand-alone RMSNorm kernel.
        if (stager) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ss = fmaf(xl[j].x, xl[j].x, ss);
                ss = fmaf(xl[j].y, xl[j].y, ss);
                ss = fmaf(xl[j].z, xl[j].z, ss);
                ss = fmaf(xl[j].w, xl[j].w, ss);
            }
            ss = wave_sum(ss);
            if (lane == 0) ssq[chunk] = ss;
        }
        __syncthreads();                                     // 0
        if (stager) {
            float tot = 0.0f;
            for (int c = 0; c < S; ++c) tot += ssq[c];
            const float inv =
                1.0f / static_cast<float>(sqrt(static_cast<double>(tot / static_cast<float>(h.K) + a.eps)));
#pragma unroll
            for (int j = 0; j < 8; ++j) xl[j] = (xl[j] * inv) * xm[j];
        }
    }

    // Stage x: float4 f of chunk c at slot c*512 + (f/8)*8 + ((f%8) ^ ((f/8)%8)).
    if (stager) {
        f32x4 *win = xwin + chunk * 512;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int f = 64 * j + lane;
            win[(f >> 3) * 8 + ((f & 7) ^ ((f >> 3) & 7))] = xl[j];
        }
    }
    __syncthreads();                                         // 1: table built, x staged
    // Epilogue operands that the last phase would otherwise fetch after the
    // row sums (one dependent memory round trip at the end of every wave):
    // the residual rows (kEAdd) and the RoPE position (kERopeKV; its cos/sin
    // pair, split-half RoPE with the stand-alone RoPE kernel's arithmetic
    // (GGUFVectorOps.rope :383-440), is requested at mid-loop once the
    // position has arrived). Each output element belongs to one finishing
    // lane, so reading it early is the same read.
    const int r = row0 + lane;
    const bool finisher = chunk == 0 && lane < T && r < row_end;
    float y_old = 0.0f;
    int rope_p = 0;
    float rope_c = 1.0f, rope_s = 0.0f;
    if constexpr (EPI == kEAdd) {
        if (finisher) {
            const RowRef f = row_ref<EPI, T>(h, r);
            y_old = seg_pick(f, a.seg[0].y, a.seg[1].y, a.seg[2].y)[f.local];
        }
    }
    if constexpr (EPI == kERopeKV) rope_p = a.pos[0];
    float xv[32];
    {
        const f32x4 *win = xwin + chunk * 512;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int f = x_f4<FMT>(lane, i);
            const f32x4 v = win[(f >> 3) * 8 + ((f & 7) ^ ((f >> 3) & 7))];
            xv[4 * i + 0] = v.x;
            xv[4 * i + 1] = v.y;
            xv[4 * i + 2] = v.z;
            xv[4 * i + 3] = v.w;
        }
    }
    float xsum = 0.0f, xsum2 = 0.0f;
    if constexpr (kquant_fmt(FMT)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xsum += xv[i];
            xsum2 += xv[16 + i];
        }
    }

    const char *tbl = reinterpret_cast<const char *>(smem);
    const uint32_t cl = (lane & 31) * 8;
    // Q4_0/Q8_0 realignment selector (v_perm): odd lanes' codes start at
    // dw[1], even lanes' 2 bytes into dw[0].
    const uint32_t align_sel = (lane & 1) ? 0x07060504u : 0x05040302u;
    float acc[TP];
#pragma unroll
    for (int t = T; t < TP; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t + PF < T && t + PF >= P0)
            load_row<FMT, EPI, T>(rw[t + PF], h, a, min(row0 + (t + PF) * rstride, row_end - 1), chunk, lo);
        if constexpr (EPI == kERopeKV) {
            if (t == T / 2 && finisher && (lane & 1) == 0) {
                const RowRef f = row_ref<EPI, T>(h, r);
                const int hd = 1 << h.hd_shift;
                if (!f.s2) rope_angle(a.rope_cs, a.cap, rope_p, f.local & (hd - 1), hd, a.rope_base, rope_c, rope_s);
            }
        }
        float scale;
        const float dot = row_dot<FMT>(rw[t], xv, xsum, xsum2, align_sel, cl, tbl, scale);
        acc[t] = dot * scale;
        // Keep the written pipeline: without these the compiler defers every
        // row's arithmetic to the end and holds all lookups in registers.
        asm volatile("" : "+v"(acc[t]));
        __builtin_amdgcn_sched_barrier(0);
    }
    const float tot = wave_sum_rows<TP>(acc);
    if (lane < TP) part[wave][wave_rows_index<TP>(lane)] = tot;
    __syncthreads();                                         // 2: partials written
    // The S chunk waves of group g are waves g*S .. g*S+S-1.
    if (finisher) {
        float v = 0.0f;
        for (int c = 0; c < S; ++c) v += part[grp * S + c][lane];
        if constexpr (EPI == kEStore || EPI == kEStore3 || EPI == kEAdd) {
            const RowRef f = row_ref<EPI, T>(h, r);
            float *y = seg_pick(f, a.seg[0].y, a.seg[1].y, a.seg[2].y);
            if constexpr (EPI == kEAdd) y[f.local] = y_old + v;
            else y[f.local] = v;
        } else if constexpr (EPI == kESwiGLU) {
            // Lane t < T/2 holds gate row i, lane t + T/2 up row i.
            if (lane < T / 2) {
                float u = 0.0f;
                for (int c = 0; c < S; ++c) u += part[grp * S + c][lane + T / 2];
                a.seg[0].y[row_ref<EPI, T>(h, r).local] = a.gelu ? geglu_metal(v, u) : silu_ref(v) * u;
            }
        } else if ((lane & 1) == 0) {
            // RoPE pairs (r, r + 1): T is even and row0 even, so both are this
            // wave's, and N is even.
            float v1 = 0.0f;
            for (int c = 0; c < S; ++c) v1 += part[grp * S + c][lane + 1];
            {
                const RowRef f = row_ref<EPI, T>(h, r);
                const int p = rope_p;
                const bool in_cache = p >= 0 && p < a.cap;
                const int hd = 1 << h.hd_shift;
                const int hh = f.local >> h.hd_shift, i = f.local & (hd - 1);
                if (!f.s1 && !f.s2) {                    // q: rotate, store fp32
                    rope_apply(v, v1, rope_c, rope_s);
                    a.seg[0].y[f.local] = v;
                    a.seg[0].y[f.local + (hd >> 1)] = v1;
                } else if (!f.s2) {                      // k: rotate, append fp16
                    rope_apply(v, v1, rope_c, rope_s);
                    if (in_cache) {
                        uint16_t *dst = a.kc + (static_cast<size_t>(hh) * a.cap + p) * hd + i;
                        dst[0] = f32_to_f16_bits(v);
                        dst[hd >> 1] = f32_to_f16_bits(v1);
                    }
                } else if (in_cache) {                   // v: rows local, local + 1, append fp16
                    uint16_t *dst = a.vc + (static_cast<size_t>(hh) * a.cap + p) * hd + i;
                    dst[0] = f32_to_f16_bits(v);
                    dst[1] = f32_to_f16_bits(v1);
                }
            }
        }
    }
}

template <int FMT, int T, int PF, int W, int XOP, int EPI, int P0>
__global__ __launch_bounds__(W * 64) void rows_kernel(const float *x, const uint8_t *w0, const float *s0,
                                                      const uint8_t *w1, const float *s1, int N, int end0, int end1,
                                                      int shape, RowsArgs a) {
    rows_body<FMT, T, PF, W, XOP, EPI, P0>(rows_hot(x, w0, s0, w1, s1, N, end0, end1, shape), a, blockIdx.x, 0, N);
}

// Two row formats in one launch (8 waves): workgroups [0, nb0) take the
// stacked rows [0, end1) in format F0, T0 rows per wave, the rest take
// [end1, N) in format F1, T1 rows per wave; the branch is per workgroup. Q
// and K of one type beside V of another (a Q4_K_M model's Q6_K V) then share
// one activation staging, RMSNorm and launch. nb0 rides in the shape word's
// bits 18 and up, so the branch waits for no argument read.
template <int F0, int T0, int PF0, int F1, int T1, int PF1, int XOP, int EPI>
__global__ __launch_bounds__(512) void rows_mix_kernel(const float *x, const uint8_t *w0, const float *s0,
                                                       const uint8_t *w1, const float *s1, int N, int end0, int end1,
                                                       int shape, RowsArgs a) {
    const RowsHot h = rows_hot(x, w0, s0, w1, s1, N, end0, end1, shape);
    const int nb0 = static_cast<int>(static_cast<unsigned>(shape) >> 18);
    const unsigned blk = blockIdx.x;
    if (blk < static_cast<unsigned>(nb0)) rows_body<F0, T0, PF0, 8, XOP, EPI, PF0>(h, a, blk, 0, end1);
    else rows_body<F1, T1, PF1, 8, XOP, EPI, PF1>(h, a, blk - nb0, end1, N);
}

template <int FMT, int T, int PF, int W, int XOP, int EPI, int P0 = PF>
void launch_cfg(const RowsArgs &args, hipStream_t s) {
    const void *fn = reinterpret_cast<const void *>(rows_kernel<FMT, T, PF, W, XOP, EPI, P0>);
    constexpr int TP = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : T <= 16 ? 16 : 32;
    const size_t lds = kLdsBytes + (W * TP + 8) * sizeof(float);
    static bool lds_set = false;                 // the attribute is per kernel, per process
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        lds_set = true;
    }
    const int rows_per_wg = args.G * T;
    const dim3 grid((args.N + rows_per_wg - 1) / rows_per_wg), block(W * 64);
    hipLaunchKernelGGL((rows_kernel<FMT, T, PF, W, XOP, EPI, P0>), grid, block, lds, s, args.x, args.seg[0].w,
                       args.seg[0].absmax, args.seg[1].w, args.seg[1].absmax, args.N, args.seg[0].end, args.seg[1].end,
                       rows_shape_word(args), args);
}

// T rows per wave (2..32), 8 waves; loads PF rows ahead: 3 when a wave's
// chunk row is most of its row (S <= 2), 4 for longer rows; Q4_0 and Q4_K
// 2 and (Q4_K) 3 (measured on the Llama MLP shapes, 14336 x 4096 and
// 4096 x 14336: Q4_0 8.67 -> 8.40 us, Q4_K 9.3 -> 8.95 and 11.0 -> 10.8 us).
template <int FMT, int XOP, int EPI, int PF>
void launch_rows_pf(const RowsArgs &args, int T, hipStream_t s) {
    switch (T) {
    case 32: launch_cfg<FMT, 32, PF, 8, XOP, EPI>(args, s); break;
    case 28: launch_cfg<FMT, 28, PF, 8, XOP, EPI>(args, s); break;
    case 24: launch_cfg<FMT, 24, PF, 8, XOP, EPI>(args, s); break;
    case 20: launch_cfg<FMT, 20, PF, 8, XOP, EPI>(args, s); break;
    case 16: launch_cfg<FMT, 16, PF, 8, XOP, EPI>(args, s); break;
    case 14: launch_cfg<FMT, 14, PF, 8, XOP, EPI>(args, s); break;
    case 12: launch_cfg<FMT, 12, PF, 8, XOP, EPI>(args, s); break;
    case 10: launch_cfg<FMT, 10, PF, 8, XOP, EPI>(args, s); break;
    case 8: launch_cfg<FMT, 8, PF, 8, XOP, EPI>(args, s); break;
    case 7: launch_cfg<FMT, 7, PF, 8, XOP, EPI>(args, s); break;
    case 6: launch_cfg<FMT, 6, PF, 8, XOP, EPI>(args, s); break;
    case 4: launch_cfg<FMT, 4, 2, 8, XOP, EPI>(args, s); break;
    default: launch_cfg<FMT, 2, 2, 8, XOP, EPI>(args, s); break;
    }
}

template <int FMT, int XOP, int EPI>
void launch_rows(RowsArgs args, int T, hipStream_t s) {
    args.G = 8 / args.S;
    constexpr int kPfShort = FMT == kFmtQ4 || FMT == kFmtQ4K ? 2 : 3;
    constexpr int kPfLong = FMT == kFmtQ4K ? 3 : 4;
    if (args.S <= 2) launch_rows_pf<FMT, XOP, EPI, kPfShort>(args, T, s);
    else launch_rows_pf<FMT, XOP, EPI, kPfLong>(args, T, s);
}

// Rows per wave: the per-workgroup set-up (activation staging, the 64 KiB
// pair table) is paid once per workgroup, and measured on MI355X the fastest
// shape is one 8-wave workgroup per CU, each taking N/CUs rows: T =
// ceil(N / (G * CUs)) rounded up to even (to a multiple of 4 above 16), at
// most `cap` (beyond that more workgroups).
int pick_rows_t(int N, int S, int cap) {
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const long long per = static_cast<long long>(8 / S) * cus;
    int t = static_cast<int>((N + per - 1) / per);
    t = (t + 1) & ~1;
    if (t > 16) t = (t + 3) & ~3;
    return t < 2 ? 2 : t > cap ? cap : t;
}

bool rows_shape_ok(const float *A, int K) {
    const int S = K / kChunk;
    return K % kChunk == 0 && S >= 1 && S <= 8 && aligned(A, 16);
}


// The batch-1 structure for MT = 2..4 NF4 tokens (a short prompt chunk or a
// small decode batch) in fp32: the same rows, pair table and activation
// staging, and every code byte's table lookup feeds the FMAs of all MT
// tokens, so the weights stream once and each token costs one FMA per
// weight. The activations of a round of R = 8/S tokens are staged together,
// one token per row group; K chunks of the MT tokens live in registers.
template <int T, int PF, int MT>
__global__ __launch_bounds__(512) void rows_mt_kernel(RowsArgs a) {
    constexpr int W = 8;
    constexpr int TP = T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : T <= 16 ? 16 : 32;
    static_assert(MT >= 2 && MT <= 4 && T <= 32, "tile shape");
    extern __shared__ float4 smem[];
    float *part = reinterpret_cast<float *>(reinterpret_cast<char *>(smem) + kLdsBytes);   // [W][MT][TP]
    f32x4 *xwin = reinterpret_cast<f32x4 *>(reinterpret_cast<char *>(smem) + kMainBytes);
    float2 *tbl2 = reinterpret_cast<float2 *>(smem);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S = a.S;
    const int chunk = wave % S;
    const int grp = wave / S;
    const int R = 8 / S;                         // tokens staged per round (one per row group)
    const int rounds = (MT + R - 1) / R;
    const bool helper = grp >= a.G;
    const int row0 = (blockIdx.x * a.G + grp) * T;
    const int xoff = chunk * kChunk;

    // Round 0's activations first, then the weight prologue.
    f32x4 xl[8];
    const bool stage0 = !helper && grp < MT;
    if (stage0) {
        const f32x4 *xw = reinterpret_cast<const f32x4 *>(a.x + static_cast<size_t>(grp) * a.K + xoff);
#pragma unroll
        for (int j = 0; j < 8; ++j) xl[j] = xw[64 * j + lane];
    }
    const LaneOffsets lo = lane_offsets<kFmtNF4>(lane, a.bs_shift);
    const RowsHot h = rows_hot(a);
    RowWords<kFmtNF4> rw[T];
    if (!helper) {
#pragma unroll
        for (int t = 0; t < PF && t < T; ++t) load_row<kFmtNF4, kEStore, T>(rw[t], h, a, min(row0 + t, a.N - 1), chunk, lo);
    }
    build_pair_table<kFmtNF4, W * 64>(tbl2, tid);

    float xv[MT][32];
    for (int rd = 0; rd < rounds; ++rd) {
        const int m = rd * R + grp;              // the token this wave stages
        const bool stager = !helper && grp < R && m < MT;
        if (stager) {
            if (rd > 0) {
                const f32x4 *xw = reinterpret_cast<const f32x4 *>(a.x + static_cast<size_t>(m) * a.K + xoff);
#pragma unroll
                for (int j = 0; j < 8; ++j) xl[j] = xw[64 * j + lane];
            }
            // Token slot grp of this round, chunk `chunk`: 512 float4s,
            // swizzled as in rows_kernel (conflict-free both ways).
            f32x4 *win = xwin + (grp * S + chunk) * 512;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int f = 64 * j + lane;
                win[(f >> 3) * 8 + ((f & 7) ^ ((f >> 3) & 7))] = xl[j];
            }
        }
        __syncthreads();
        if (!helper) {
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                if (mm / R != rd) continue;      // uniform: staged in another round
                const f32x4 *win = xwin + ((mm % R) * S + chunk) * 512;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int f = lane * 8 + i;
                    const f32x4 v = win[(f >> 3) * 8 + ((f & 7) ^ ((f >> 3) & 7))];
                    xv[mm][4 * i + 0] = v.x;
                    xv[mm][4 * i + 1] = v.y;
                    xv[mm][4 * i + 2] = v.z;
                    xv[mm][4 * i + 3] = v.w;
                }
            }
        }
        if (rd + 1 < rounds) __syncthreads();    // the next round overwrites the windows
    }

    if (!helper) {
        const uint32_t cl = (lane & 31) * 8;
        float acc[MT][TP];
#pragma unroll
        for (int mm = 0; mm < MT; ++mm)
#pragma unroll
            for (int t = 0; t < TP; ++t) acc[mm][t] = 0.0f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            if (t + PF < T) load_row<kFmtNF4, kEStore, T>(rw[t + PF], h, a, min(row0 + t + PF, a.N - 1), chunk, lo);
            const uint32_t wv[4] = {rw[t].q.x, rw[t].q.y, rw[t].q.z, rw[t].q.w};
            float p0[MT], p1[MT];
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) p0[mm] = p1[mm] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float2 e[4];
                e[0] = pair_at(nullptr, pair_addr<0>(wv[i], cl));
                e[1] = pair_at(nullptr, pair_addr<1>(wv[i], cl));
                e[2] = pair_at(nullptr, pair_addr<2>(wv[i], cl));
                e[3] = pair_at(nullptr, pair_addr<3>(wv[i], cl));
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int mm = 0; mm < MT; ++mm) {
                        p0[mm] = fmaf(e[b].x, xv[mm][8 * i + 2 * b], p0[mm]);
                        p1[mm] = fmaf(e[b].y, xv[mm][8 * i + 2 * b + 1], p1[mm]);
                    }
            }
#pragma unroll
            for (int mm = 0; mm < MT; ++mm) {
                acc[mm][t] = (p0[mm] + p1[mm]) * rw[t].s;
                asm volatile("" : "+v"(acc[mm][t]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            const float tot = wave_sum_rows<TP>(acc[mm]);
            if (lane < TP) part[(wave * MT + mm) * TP + wave_rows_index<TP>(lane)] = tot;
        }
    }
    __syncthreads();
    const int r = row0 + lane;
    if (!helper && chunk == 0 && lane < T && r < a.N) {
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            float v = 0.0f;
            for (int c = 0; c < S; ++c) v += part[((grp * S + c) * MT + mm) * TP + lane];
            a.seg[0].y[static_cast<size_t>(mm) * a.N + r] = v;
        }
    }
}

template <int T, int PF, int MT>
void launch_mt_cfg(const RowsArgs &args, hipStream_t s) {
    const void *fn = reinterpret_cast<const void *>(rows_mt_kernel<T, PF, MT>);
    constexpr int TP = T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : T <= 16 ? 16 : 32;
    const size_t lds = kLdsBytes + 8 * MT * TP * sizeof(float);
    static bool lds_set = false;
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        lds_set = true;
    }
    const int rows_per_wg = args.G * T;
    hipLaunchKernelGGL((rows_mt_kernel<T, PF, MT>), dim3((args.N + rows_per_wg - 1) / rows_per_wg), dim3(512), lds,
                       s, args);
}

template <int MT>
void launch_mt(const RowsArgs &args, int T, hipStream_t s) {
    switch (T) {
    case 32: launch_mt_cfg<32, 3, MT>(args, s); break;
    case 28: launch_mt_cfg<28, 3, MT>(args, s); break;
    case 24: launch_mt_cfg<24, 3, MT>(args, s); break;
    case 20: launch_mt_cfg<20, 3, MT>(args, s); break;
    case 16: launch_mt_cfg<16, 3, MT>(args, s); break;
    case 14: launch_mt_cfg<14, 3, MT>(args, s); break;
    case 12: launch_mt_cfg<12, 3, MT>(args, s); break;
    case 10: launch_mt_cfg<10, 3, MT>(args, s); break;
    case 8: launch_mt_cfg<8, 3, MT>(args, s); break;
    case 6: launch_mt_cfg<6, 3, MT>(args, s); break;
    case 4: launch_mt_cfg<4, 2, MT>(args, s); break;
    default: launch_mt_cfg<2, 2, MT>(args, s); break;
    }
}

}  // namespace

// C[M][N] for M = 2..4 NF4 tokens (fp32, the batch-1 rows kernel's shape
// limits); ALJABR_ROCM_ERR_UNSUPPORTED for anything else.
int enqueue_rows_nf4_mt(float *C, const float *A, const uint8_t *W, const float *absmax, int K, int N, int bs_shift,
                        int M) {
    if (M < 2 || M > 4 || !rows_shape_ok(A, K) || bs_shift < 5 || bs_shift > 11 || !aligned(W, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    RowsArgs args{};
    args.seg[0] = RowsSeg{W, absmax, C, N};
    args.seg[1].end = args.seg[2].end = 0x7fffffff;
    args.x = A;
    args.N = N;
    args.K = K;
    args.bs_shift = bs_shift;
    args.S = K / kChunk;
    args.G = 8 / args.S;
    const int T = pick_rows_t(N, args.S, 16);   // MT x T accumulators stay in registers
    hipStream_t s = current_stream();
    switch (M) {
    case 2: launch_mt<2>(args, T, s); break;
    case 3: launch_mt<3>(args, T, s); break;
    default: launch_mt<4>(args, T, s); break;
    }
    return ALJABR_ROCM_OK;
}

namespace {
}  // namespace

int enqueue_rows(float *C, const float *A, const uint8_t *W, const float *absmax, int K, int N, int type,
                 int bs_shift) {
    if (!rows_shape_ok(A, K)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    int fmt;
    if (type == ALJABR_ROCM_TYPE_NF4) {
        // Blocks of 32 .. 2048 weights: a lane's 32 weights share one absmax
        // and a chunk's blocks start on its first weight.
        if (bs_shift < 5 || bs_shift > 11 || !aligned(W, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
        fmt = kFmtNF4;
    } else if (type == ALJABR_ROCM_TYPE_Q4_0 || type == ALJABR_ROCM_TYPE_Q8_0) {
        if (!aligned(W, 4)) return ALJABR_ROCM_ERR_UNSUPPORTED;
        fmt = type == ALJABR_ROCM_TYPE_Q4_0 ? kFmtQ4 : kFmtQ8;
    } else if (type == ALJABR_ROCM_TYPE_Q4_K || type == ALJABR_ROCM_TYPE_Q6_K) {
        if (!aligned(W, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
        fmt = type == ALJABR_ROCM_TYPE_Q4_K ? kFmtQ4K : kFmtQ6K;
    } else {
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    }
    RowsArgs args{};
    args.seg[0] = RowsSeg{W, absmax, C, N};
    args.seg[1].end = args.seg[2].end = 0x7fffffff;
    args.x = A;
    args.N = N;
    args.K = K;
    args.bs_shift = bs_shift;
    args.S = K / kChunk;
    const int T = pick_rows_t(N, args.S, 16);
    hipStream_t s = current_stream();
    switch (fmt) {
    case kFmtNF4: launch_rows<kFmtNF4, kXPlain, kEStore>(args, T, s); break;
    case kFmtQ4: launch_rows<kFmtQ4, kXPlain, kEStore>(args, T, s); break;
    case kFmtQ4K: launch_rows<kFmtQ4K, kXPlain, kEStore>(args, T, s); break;
    case kFmtQ6K: launch_rows<kFmtQ6K, kXPlain, kEStore>(args, T, s); break;
    default: launch_rows<kFmtQ8, kXPlain, kEStore>(args, T, s); break;
    }
    return ALJABR_ROCM_OK;
}

namespace {

template <int FMT>
int launch_fused(RowsArgs &args, int T, int epilogue, bool norm, hipStream_t s) {
    switch (epilogue) {
    case kRowsStore:
        if (args.seg[1].end < args.N) {          // three segments
            if (norm) launch_rows<FMT, kXNorm, kEStore3>(args, T, s);
            else launch_rows<FMT, kXPlain, kEStore3>(args, T, s);
        } else {
            if (norm) launch_rows<FMT, kXNorm, kEStore>(args, T, s);
            else launch_rows<FMT, kXPlain, kEStore>(args, T, s);
        }
        return ALJABR_ROCM_OK;
    case kRowsAdd:
        if (norm) return ALJABR_ROCM_ERR_UNSUPPORTED;
        launch_rows<FMT, kXPlain, kEAdd>(args, T, s);
        return ALJABR_ROCM_OK;
    case kRowsSwiGLU:
    case kRowsGeGLU:
        if (!norm) return ALJABR_ROCM_ERR_UNSUPPORTED;
        args.gelu = epilogue == kRowsGeGLU;
        launch_rows<FMT, kXNorm, kESwiGLU>(args, T, s);
        return ALJABR_ROCM_OK;
    default:
        if (!norm) return ALJABR_ROCM_ERR_UNSUPPORTED;
        launch_rows<FMT, kXNorm, kERopeKV>(args, T, s);
        return ALJABR_ROCM_OK;
    }
}

}  // namespace

int enqueue_nf4_rows_fused(const RowsOut *outs, int nseg, const float *x, const float *norm_w, float eps, int K,
                           int bs_shift, int epilogue, const RowsRope *rope) {
    return enqueue_rows_fused(ALJABR_ROCM_TYPE_NF4, outs, nseg, x, norm_w, eps, K, bs_shift, epilogue, rope);
}

namespace {

// The launch arguments of a fused rows launch (segments, epilogue operands,
// shape), or UNSUPPORTED.
int fused_args(int type, const RowsOut *outs, int nseg, const float *x, const float *norm_w, float eps, int K,
               int bs_shift, int epilogue, const RowsRope *rope, RowsArgs &args) {
    if (nseg < 1 || nseg > 3 || !rows_shape_ok(x, K)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (type == ALJABR_ROCM_TYPE_NF4 && (bs_shift < 5 || bs_shift > 11)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (type != ALJABR_ROCM_TYPE_NF4 && type != ALJABR_ROCM_TYPE_Q4_0 && type != ALJABR_ROCM_TYPE_Q8_0 &&
        type != ALJABR_ROCM_TYPE_Q4_K && type != ALJABR_ROCM_TYPE_Q6_K)
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (norm_w && !aligned(norm_w, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args = RowsArgs{};
    if (epilogue == kRowsSwiGLU || epilogue == kRowsGeGLU) {
        // gate (segment 0) and up (segment 1) interleaved row by row.
        if (nseg != 2 || outs[0].n != outs[1].n) return ALJABR_ROCM_ERR_UNSUPPORTED;
    } else if (epilogue == kRowsRopeKV) {
        // q, k, v of one sequence; RoPE pairs of q and k meet in one wave.
        // Segments may be empty (n = 0), so that q, k and v of different
        // types take one launch per type: the rows of an empty segment are
        // never formed.
        // k and v rows address cache head local / head_dim, so both hold
        // whole heads, at most n_kv of them, and the same count when a launch
        // carries both.
        const int hs = rope ? log2_exact(rope->head_dim) : -1;
        if (nseg != 3 || !rope || !rope->pos || !rope->kc || !rope->vc || hs < 1 || rope->n_kv < 1 ||
            outs[0].n < 0 || outs[1].n < 0 || outs[2].n < 0 || outs[0].n % rope->head_dim != 0 ||
            outs[1].n % rope->head_dim != 0 || outs[2].n % rope->head_dim != 0 ||
            outs[1].n / rope->head_dim > rope->n_kv || outs[2].n / rope->head_dim > rope->n_kv ||
            (outs[1].n > 0 && outs[2].n > 0 && outs[1].n != outs[2].n) || outs[0].n + outs[1].n + outs[2].n == 0)
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        args.pos = rope->pos;
        args.kc = rope->kc;
        args.vc = rope->vc;
        args.cap = rope->cap;
        args.hd_shift = hs;
        args.rope_base = rope->base;
        args.rope_cs = rope->cs;
    } else if (epilogue != kRowsStore && epilogue != kRowsAdd) {
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    }
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const size_t wa = (type == ALJABR_ROCM_TYPE_Q4_0 || type == ALJABR_ROCM_TYPE_Q8_0) ? 4 : 16;
            // Only the RoPE epilogue takes empty segments (checked above).
            const bool empty_ok = epilogue == kRowsRopeKV && outs[i].n == 0;
            if (!empty_ok && (!aligned(outs[i].w, wa) || outs[i].n <= 0 || (outs[i].n & 1)))
                return ALJABR_ROCM_ERR_UNSUPPORTED;
            end += outs[i].n;
            if (end > 0x7ffffffeLL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.seg[i] = RowsSeg{outs[i].w, outs[i].absmax, outs[i].y, static_cast<int>(end)};
        } else {
            args.seg[i].end = 0x7fffffff;
        }
    }
    args.x = x;
    args.norm_w = norm_w;
    args.eps = eps;
    args.N = static_cast<int>(end);
    args.K = K;
    args.bs_shift = bs_shift;
    args.S = K / kChunk;
    args.G = 8 / args.S;
    return ALJABR_ROCM_OK;
}

template <int F0, int T0, int F1, int T1, int EPI>
void launch_mix(const RowsArgs &args, int nb0, int nb1, hipStream_t s) {
    constexpr int PF0 = T0 <= 4 ? 2 : 3, PF1 = T1 <= 4 ? 2 : 3;
    constexpr int TPM = T0 > T1 ? (T0 <= 4 ? 4 : 8) : (T1 <= 4 ? 4 : 8);
    const void *fn = reinterpret_cast<const void *>(rows_mix_kernel<F0, T0, PF0, F1, T1, PF1, kXNorm, EPI>);
    static bool lds_set = false;                 // the attribute is per kernel, per process
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        lds_set = true;
    }
    const size_t lds = kLdsBytes + (8 * TPM + 8) * sizeof(float);
    hipLaunchKernelGGL((rows_mix_kernel<F0, T0, PF0, F1, T1, PF1, kXNorm, EPI>), dim3(nb0 + nb1), dim3(512), lds,
                       s, args.x, args.seg[0].w, args.seg[0].absmax, args.seg[1].w, args.seg[1].absmax, args.N,
                       args.seg[0].end, args.seg[1].end, rows_shape_word(args) | (nb0 << 18), args);
}

template <int F0, int F1, int T0, int EPI>
void launch_mix_t1(const RowsArgs &args, int T1, int nb0, int nb1, hipStream_t s) {
    if (T1 == 2) launch_mix<F0, T0, F1, 2, EPI>(args, nb0, nb1, s);
    else if (T1 == 4) launch_mix<F0, T0, F1, 4, EPI>(args, nb0, nb1, s);
    else launch_mix<F0, T0, F1, 8, EPI>(args, nb0, nb1, s);
}

template <int EPI>
void launch_mix_t0(const RowsArgs &args, int T0, int T1, int nb0, int nb1, hipStream_t s) {
    switch (T0) {
    case 2: launch_mix_t1<kFmtQ4K, kFmtQ6K, 2, EPI>(args, T1, nb0, nb1, s); break;
    case 4: launch_mix_t1<kFmtQ4K, kFmtQ6K, 4, EPI>(args, T1, nb0, nb1, s); break;
    case 6: launch_mix_t1<kFmtQ4K, kFmtQ6K, 6, EPI>(args, T1, nb0, nb1, s); break;
    default: launch_mix_t1<kFmtQ4K, kFmtQ6K, 8, EPI>(args, T1, nb0, nb1, s); break;
    }
}

}  // namespace

// Q and K (segments 0 and 1) in Q4_K beside V (segment 2) in Q6_K: RMSNorm
// and the products in one launch, with RoPE and the cache append
// (kRowsRopeKV) or stored (kRowsStore). T0 is the one-type launch's rows per
// wave for the first two segments; T1 (2, 4 or 8) the smallest that keeps
// both parts' workgroups within one per CU. UNSUPPORTED for other types,
// epilogues or shapes (the caller then launches per type).
int enqueue_rows_mixed(int type01, int type2, const RowsOut *outs, const float *x, const float *norm_w, float eps,
                       int K, int epilogue, const RowsRope *rope) {
    if (type01 != ALJABR_ROCM_TYPE_Q4_K || type2 != ALJABR_ROCM_TYPE_Q6_K || !norm_w ||
        (epilogue != kRowsRopeKV && epilogue != kRowsStore))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (outs[0].n <= 0 || outs[1].n <= 0 || outs[2].n <= 0) return ALJABR_ROCM_ERR_UNSUPPORTED;
    RowsArgs args;
    const int rc = fused_args(type01, outs, 3, x, norm_w, eps, K, 0, epilogue, rope, args);
    if (rc != ALJABR_ROCM_OK) return rc;
    if (args.S > 2) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int n0 = args.seg[1].end, n1 = args.N - n0;
    const int T0 = pick_rows_t(n0, args.S, 8);   // even, 2..8
    const int nb0 = (n0 + args.G * T0 - 1) / (args.G * T0);
    int T1 = 0, nb1 = 0;
    for (int t = 2; t <= 8; t *= 2) {
        nb1 = (n1 + args.G * t - 1) / (args.G * t);
        if (nb0 + nb1 <= cus) {
            T1 = t;
            break;
        }
    }
    if (!T1 || nb0 >= (1 << 13)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    hipStream_t s = current_stream();
    if (epilogue == kRowsRopeKV) launch_mix_t0<kERopeKV>(args, T0, T1, nb0, nb1, s);
    else launch_mix_t0<kEStore3>(args, T0, T1, nb0, nb1, s);
    return ALJABR_ROCM_OK;
}

int enqueue_rows_fused(int type, const RowsOut *outs, int nseg, const float *x, const float *norm_w, float eps, int K,
                       int bs_shift, int epilogue, const RowsRope *rope) {
    RowsArgs args;
    const int rc = fused_args(type, outs, nseg, x, norm_w, eps, K, bs_shift, epilogue, rope, args);
    if (rc != ALJABR_ROCM_OK) return rc;
    int T = pick_rows_t(args.N, args.S, 32);
    if (T & 1) ++T;                              // the paired epilogues need both rows of a pair in one wave
    if ((epilogue == kRowsSwiGLU || epilogue == kRowsGeGLU) && (outs[0].n % (T / 2)) != 0)
        return ALJABR_ROCM_ERR_UNSUPPORTED;      // every wave's gate run must be whole
    hipStream_t s = current_stream();
    const bool norm = norm_w != nullptr;
    switch (type) {
    case ALJABR_ROCM_TYPE_NF4: return launch_fused<kFmtNF4>(args, T, epilogue, norm, s);
    case ALJABR_ROCM_TYPE_Q4_0: return launch_fused<kFmtQ4>(args, T, epilogue, norm, s);
    case ALJABR_ROCM_TYPE_Q8_0: return launch_fused<kFmtQ8>(args, T, epilogue, norm, s);
    case ALJABR_ROCM_TYPE_Q4_K: return launch_fused<kFmtQ4K>(args, T, epilogue, norm, s);
    default: return launch_fused<kFmtQ6K>(args, T, epilogue, norm, s);
    }
}

}  // namespace aljabr
