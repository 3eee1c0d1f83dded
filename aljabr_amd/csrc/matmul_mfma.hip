// matmul_mfma.hip - NF4 small-M GEMM on the matrix cores, deterministic:
// Y[M,N] = X[M,K] . W[N,K]^T (or Y += ...) for passes of up to 64 tokens (a
// prompt chunk or a decode batch), W in NF4
// (STC/DequantizationKernel.java:84-102). Replaces the reference's per-token
// loop over the matvec (MTLJ/MetalComputeBackend.java:435-470): W is read
// from HBM once for all tokens of a pass.
//
// Two kernels: nf4_gemm_kernel (below the first one; K % 1024 == 0) keeps
// the activations in registers and is the one the decode step and the
// batched ABI run; nf4_mm_kernel, described here, stages them in LDS and
// takes the other shapes (K % 256 == 0).
//
// Precision. MFMA v_mfma_f32_32x32x16_f16 with A = X (32 token rows) and
// B = W^T (32 weight rows per wave as the output columns), fp32 accumulation.
// Neither operand is rounded: activations are split x = xh + xl (xh =
// fp16(x), xl = fp16(x - xh)) and NF4 levels L = H + R (H = fp16(L),
// R = fp16(L - H)), and each product is xh.H + xl.H + xh.R; the dropped
// xl.R term and the fp16 rounding of R are below 2^-22 of the product. The
// per-64-element absmax multiplies the fp32 accumulators once per block.
//
// Decode. A code byte (two weights) indexes a 256-entry LDS table holding
// the byte's H pair and R pair (the hi and lo B registers), replicated 32
// times: the H pair of replica r at byte e*256 + 4r, the R pair at
// e*256 + 128 + 4r, so the 32 lanes of a half-wave read 32 distinct banks.
// The address is one v_perm_b32 of the code dword and the lane's offset.
//
// Work split. A workgroup is 8 waves; wave w owns 32 rows of the
// workgroup's 256-row group and runs a slice of consecutive 256-element K
// sub-slices. Weight codes are loaded coalesced (8 lanes per 128-byte row
// segment), four sub-slices ahead in registers, and turned into the MFMA B
// layout through a per-wave LDS stage; each sub-slice's activations (hi and
// lo) are staged once per workgroup in LDS.
//
// Determinism. With several K slices, each workgroup stores its partial
// tile and a second kernel sums the slices in slice order into Y (or adds
// them to it): no float atomics, the same result on every run.
#include <atomic>
#include <type_traits>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));

constexpr int kMmWaves = 8;
constexpr int kMmThreads = kMmWaves * 64;
constexpr int kGroupRows = kMmWaves * 32;        // rows of a workgroup
constexpr int kSub = 256;                        // K sub-slice (elements) staged at a time
constexpr int kRS = kSub + 8;                    // activation row stride in halves (16-byte pad)

// LDS layout (bytes; dynamic LDS starts at address 0, the kernel has no
// static LDS): the decode table, the activation tile of MT 32-token tiles
// (hi rows, then lo rows), per-wave code staging (32 rows x 144 bytes) and
// per-wave scale staging (32 rows x 4 floats). With two token tiles the
// table keeps 16 replicas in 128-byte entries (32 KiB) so that the 64
// activation rows fit.
constexpr uint32_t kCRow = 144;
template <int MT>
struct Lds {
    static constexpr uint32_t kReplicas = MT == 1 ? 32 : 16;
    static constexpr uint32_t kEntry = 8 * kReplicas;                 // H pairs, then R pairs
    static constexpr uint32_t kTableBytes = 256 * kEntry;
    static constexpr uint32_t kXOff = kTableBytes;
    static constexpr uint32_t kXLo = 32 * MT * kRS * 2;               // lo rows after the hi rows
    static constexpr uint32_t kCOff = kXOff + 2 * kXLo;
    static constexpr uint32_t kSOff = kCOff + kMmWaves * 32 * kCRow;
    static constexpr uint32_t kBytes = kSOff + kMmWaves * 32 * 16;
    static_assert(kBytes <= 160 * 1024, "LDS budget of a CU");
};

// Up to three weight matrices of the same K stacked as one row space (the
// decode step's Q/K/V or gate/up in one launch): segment s owns stacked rows
// [end[s-1], end[s]); every segment but the last holds a multiple of 32 rows,
// so a 32-row tile never straddles two.
struct MmArgs {
    float *y[3];
    const float *x;
    const uint8_t *w[3];
    const float *absmax[3];
    int end[3];
    int nseg;
    int M, N, K;           // N: stacked rows
    int add;               // Y += instead of Y = (one slice)
    int q;                 // sub-slices per slice (the last slice may hold fewer)
    float *part;           // [slice][M][N] partial sums (several slices, or a tail kernel follows); null: Y directly
};

struct TileRef {
    const uint8_t *w;
    const float *absmax;
    float *y;
    int local0, n;
};

__device__ __forceinline__ int segment_of(const int (&end)[3], int nseg, int r) {
    const int s = (r >= end[0]) + (r >= end[1]);
    return s > nseg - 1 ? nseg - 1 : s;
}

// An argument value pinned in scalar registers: selecting between pinned
// values stays a select (folded into one load at a computed address, the
// argument block would be copied to scratch memory).
template <typename T>
__device__ __forceinline__ T pin(T v) {
    asm volatile("" : "+s"(v));
    return v;
}

// The segment of stacked row r0 (uniform across the wave).
__device__ __forceinline__ TileRef tile_ref(const MmArgs &a, int r0) {
    const int e0 = pin(a.end[0]), e1 = pin(a.end[1]), e2 = pin(a.end[2]);
    int s = (r0 >= e0) + (r0 >= e1);
    if (s > a.nseg - 1) s = a.nseg - 1;
    const int start = s == 0 ? 0 : s == 1 ? e0 : e1;
    TileRef t;
    t.w = s == 0 ? pin(a.w[0]) : s == 1 ? pin(a.w[1]) : pin(a.w[2]);
    t.absmax = s == 0 ? pin(a.absmax[0]) : s == 1 ? pin(a.absmax[1]) : pin(a.absmax[2]);
    t.y = s == 0 ? pin(a.y[0]) : s == 1 ? pin(a.y[1]) : pin(a.y[2]);
    t.local0 = r0 - start;
    t.n = (s == 0 ? e0 : s == 1 ? e1 : e2) - start;
    return t;
}

__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
    const _Float16 a = static_cast<_Float16>(lo), b = static_cast<_Float16>(hi);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// fp16 residual of a level: L - fp16(L), rounded to fp16.
__device__ __forceinline__ float level_rest(float l) {
    return l - static_cast<float>(static_cast<_Float16>(l));
}

typedef uint32_t __attribute__((address_space(3))) lds_u32;
typedef u32x2v __attribute__((address_space(3))) lds_u32x2;
typedef u32x4v __attribute__((address_space(3))) lds_u32x4;
typedef f32x2 __attribute__((address_space(3))) lds_f32x2;
typedef f32x4 __attribute__((address_space(3))) lds_f32x4;
typedef half8 __attribute__((address_space(3))) lds_half8;

template <typename T>
__device__ __forceinline__ T *lds(uint32_t addr) {
    return reinterpret_cast<T *>(static_cast<uintptr_t>(addr));
}

// Global-memory loads through explicitly global pointers (a pointer that
// went through a pinned register would otherwise load as FLAT, whose
// counters force full waits).
template <typename T>
__device__ __forceinline__ T gload(const void *p) {
    typedef const T __attribute__((address_space(1))) gT;
    return *(gT *)(p);
}
template <typename T>
__device__ __forceinline__ T gload_stream(const void *p) {
    typedef const T __attribute__((address_space(1))) gT;
    return __builtin_nontemporal_load((gT *)(p));
}

// Table entry e (code byte: even element in the high nibble), replica r:
// {H(e>>4), H(e&15)} at e*kEntry + 4r and {R(e>>4), R(e&15)} kEntry/2 bytes
// on. With 32 replicas thread tid (of 512) fills replica tid%32 of entries
// tid/32 + 16k, k < 16 (low nibble tid/32, high nibble k); with 16 replicas
// replica tid%16 of entries tid/16 + 32k, k < 8 (low nibble (tid/16)%16,
// high nibble tid/256 + 2k).
template <int MT>
__device__ __forceinline__ void build_table(int tid) {
    constexpr float kNF4[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
    if constexpr (MT == 1) {
        const float lo = nf4_level_sel((tid >> 5) & 15);
        const uint32_t base = static_cast<uint32_t>(tid >> 5) * 256 + (tid & 31) * 4;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float hi = kNF4[k];
            *lds<lds_u32>(base + k * 16 * 256) = pack_half2(hi, lo);
            *lds<lds_u32>(base + k * 16 * 256 + 128) = pack_half2(level_rest(hi), level_rest(lo));
        }
    } else {
        const float lo = nf4_level_sel((tid >> 4) & 15);
        const uint32_t base = static_cast<uint32_t>(tid >> 4) * 128 + (tid & 15) * 4;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float hi = nf4_level_sel(2 * k + (tid >> 8));
            *lds<lds_u32>(base + k * 32 * 128) = pack_half2(hi, lo);
            *lds<lds_u32>(base + k * 32 * 128 + 64) = pack_half2(level_rest(hi), level_rest(lo));
        }
    }
}

// B fragments (8 weights, hi and residual) of code dword `w`: byte t holds
// elements 2t (high nibble) and 2t+1 (low nibble). `ch` is the lane's H
// offset within an entry (4*(lane%32)); the R pair sits 128 bytes on and is
// read as a relaxed atomic, which keeps the two reads separate (merged into
// one paired read they would land in adjacent registers and need moves),
// so one v_perm address serves both and every read lands in its fragment
// register.
// With 16 replicas (MT = 2) `ch` is 8*(lane%16) and the permuted address is
// halved: byte*128 + 4*(lane%16), entries of 128 bytes.
template <int MT>
__device__ __forceinline__ void decode8(uint32_t w, uint32_t ch, half8 &bh, half8 &br) {
    constexpr uint32_t RO = Lds<MT>::kEntry / 2;
    const int sh = MT == 1 ? 0 : 1;
    const uint32_t a0 = __builtin_amdgcn_perm(w, ch, 0x0C0C0400u) >> sh;
    const uint32_t a1 = __builtin_amdgcn_perm(w, ch, 0x0C0C0500u) >> sh;
    const uint32_t a2 = __builtin_amdgcn_perm(w, ch, 0x0C0C0600u) >> sh;
    const uint32_t a3 = __builtin_amdgcn_perm(w, ch, 0x0C0C0700u) >> sh;
    u32x4v h, r;
    h.x = *lds<lds_u32>(a0);
    h.y = *lds<lds_u32>(a1);
    h.z = *lds<lds_u32>(a2);
    h.w = *lds<lds_u32>(a3);
    r.x = __hip_atomic_load(lds<lds_u32>(a0 + RO), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    r.y = __hip_atomic_load(lds<lds_u32>(a1 + RO), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    r.z = __hip_atomic_load(lds<lds_u32>(a2 + RO), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    r.w = __hip_atomic_load(lds<lds_u32>(a3 + RO), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    bh = __builtin_bit_cast(half8, h);
    br = __builtin_bit_cast(half8, r);
}

// One work unit: a wave's 32 weight rows x one 256-element sub-slice (128
// code bytes and 4 scales per row), loaded coalesced: load i covers rows
// 8i + lane/8, bytes 16*(lane%8) of the row's segment; the scale pair of a
// lane is row lane/2, scales 2*(lane%2) and +1.
struct Unit {
    u32x4 q[4];
    f32x2 s;
};

// A lane's load addresses for a tile at K offset 0: the four code rows it
// loads (rows 8i + lane/8, bytes 16*(lane%8)) and its scale pair (row
// lane/2, scales 2*(lane%2)); a unit at K offset k0 adds k0/2 bytes to the
// codes and k0/64 floats to the scales.
struct UnitBase {
    const uint8_t *q[4];
    const float *s;
};

__device__ __forceinline__ UnitBase unit_base(const TileRef &tr, int K, int lane) {
    const size_t row_bytes = static_cast<size_t>(K) >> 1;
    UnitBase b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = min(tr.local0 + 8 * i + (lane >> 3), tr.n - 1);
        b.q[i] = tr.w + static_cast<size_t>(row) * row_bytes + 16 * (lane & 7);
    }
    const int srow = min(tr.local0 + (lane >> 1), tr.n - 1);
    b.s = tr.absmax + static_cast<size_t>(srow) * (K >> 6) + 2 * (lane & 1);
    return b;
}

// All-ones when `real`, else zero, through an opaque register so the
// compiler keeps one load instruction with a masked address (a branch per
// case would break the exact wait counts).
__device__ __forceinline__ uintptr_t real_mask(bool real) {
    uint32_t r = real ? 1u : 0u;
    asm volatile("" : "+v"(r));
    return static_cast<uintptr_t>(0) - static_cast<uintptr_t>(r);
}

// Loads of the unit at K offset k0 (uniform); a dummy unit (past the
// slice's end) loads the base of `dummy` in every lane instead: one line.
__device__ __forceinline__ void issue_unit(Unit &u, const UnitBase &b, int k0, bool real, const void *dummy) {
    const uintptr_t mask = real_mask(real), d = reinterpret_cast<uintptr_t>(dummy);
    const auto pick = [&](const void *p) {
        return reinterpret_cast<const void *>((reinterpret_cast<uintptr_t>(p) & mask) | (d & ~mask));
    };
    u.s = gload<f32x2>(pick(b.s + (k0 >> 6)));
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = gload_stream<u32x4>(pick(b.q[i] + (k0 >> 1)));
    __builtin_amdgcn_sched_barrier(0);           // keep units in issue order
}

// Activations as four float4 chunks per thread, coalesced: chunk c =
// tid + 512j is token row c/64 = tid/64 + 8j, elements 4*(tid%64) .. +4 of
// the sub-slice. Rows >= M load row 0: they only feed output rows >= M,
// which are never stored.
template <int MT>
struct XBase {
    const float *p[4 * MT];
};

template <int MT>
__device__ __forceinline__ XBase<MT> x_base(const float *x, int M, int K, int tid) {
    XBase<MT> b;
#pragma unroll
    for (int j = 0; j < 4 * MT; ++j) {
        const int m = (tid >> 6) + 8 * j;
        b.p[j] = x + static_cast<size_t>(m < M ? m : 0) * K + 4 * (tid & 63);
    }
    return b;
}

template <int MT>
__device__ __forceinline__ void load_x(f32x4 (&xr)[4 * MT], const XBase<MT> &b, int k0, bool real,
                                       const float *dummy) {
    const uintptr_t mask = real_mask(real), d = reinterpret_cast<uintptr_t>(dummy);
#pragma unroll
    for (int j = 0; j < 4 * MT; ++j)
        xr[j] = gload<f32x4>(reinterpret_cast<const void *>((reinterpret_cast<uintptr_t>(b.p[j] + k0) & mask) |
                                                            (d & ~mask)));
    // Issued where written: sunk below the MFMA work, these loads would
    // share registers with it and stall it on their return.
    __builtin_amdgcn_sched_barrier(0);
}

// Stage the activations as hi and lo halves (consecutive lanes write
// consecutive 8-byte pieces of a row): hi = fp16(x) and lo = fp16(x - hi),
// both rounded toward zero (packed conversions); x - hi is exact in fp32
// and lo keeps its leading 11 bits, below 2^-22 of x.
template <int MT>
__device__ __forceinline__ void stage_x(const f32x4 (&xr)[4 * MT], int tid) {
#pragma unroll
    for (int j = 0; j < 4 * MT; ++j) {
        const int m = (tid >> 6) + 8 * j;
        const f32x4 v = xr[j];
        typedef __fp16 half2v __attribute__((ext_vector_type(2)));
        const half2v h01 = __builtin_amdgcn_cvt_pkrtz(v.x, v.y);
        const half2v h23 = __builtin_amdgcn_cvt_pkrtz(v.z, v.w);
        const half2v l01 = __builtin_amdgcn_cvt_pkrtz(v.x - static_cast<float>(h01.x), v.y - static_cast<float>(h01.y));
        const half2v l23 = __builtin_amdgcn_cvt_pkrtz(v.z - static_cast<float>(h23.x), v.w - static_cast<float>(h23.y));
        const uint32_t addr = Lds<MT>::kXOff + (m * kRS + 4 * (tid & 63)) * 2;
        *lds<lds_u32x2>(addr) = u32x2v{__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)};
        *lds<lds_u32x2>(addr + Lds<MT>::kXLo) =
            u32x2v{__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)};
    }
}

// A unit's codes and scales in the MFMA B layout, through the wave's
// staging rows: lane (nl, h) = (lane%32, lane/32) takes bytes 32b + 16h of
// row nl for block b (elements 64b + 32h .. +32) and row nl's four scales.
// The staging rows are the wave's own and its LDS operations run in order,
// so no barrier is needed (and a second unit may reuse them at once).
__device__ __forceinline__ void to_mfma_layout(const Unit &u, u32x4v (&qm)[4], f32x4 &sc, uint32_t cst, uint32_t sst,
                                               int lane) {
    const int nl = lane & 31, h = lane >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) *lds<lds_u32x4>(cst + (8 * i + (lane >> 3)) * kCRow + 16 * (lane & 7)) = u.q[i];
    *lds<lds_f32x2>(sst + (lane >> 1) * 16 + 8 * (lane & 1)) = u.s;
#pragma unroll
    for (int b = 0; b < 4; ++b) qm[b] = *lds<lds_u32x4>(cst + nl * kCRow + 32 * b + 16 * h);
    sc = *lds<lds_f32x4>(sst + nl * 16);
}

// acc[t][mt] += blockwise-scaled product of unit t (NT units: the wave's
// row tiles, one sub-slice) with token tile mt of the staged activations.
// Each A fragment is read once for all NT row tiles and each decoded B
// fragment feeds all MT token tiles; the MFMA chains interleave. `arow` is
// the LDS address of the lane's A row plus its half in token tile 0.
template <int NT, int MT>
__device__ __forceinline__ void compute_units(f32x16 (&acc)[NT][MT], const Unit *u, uint32_t arow, uint32_t cst,
                                              uint32_t sst, int lane, uint32_t ch) {
    constexpr uint32_t kTileX = 32 * kRS * 2;     // bytes of one token tile's hi rows
    u32x4v qm[NT][4];
    f32x4 sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) to_mfma_layout(u[t], qm[t], sc[t], cst, sst, lane);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        f32x16 cb[NT][MT];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = arow + (64 * b + 8 * j) * 2;
            half8 ah[MT], al[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                ah[mt] = *lds<lds_half8>(e + mt * kTileX);
                al[mt] = *lds<lds_half8>(e + mt * kTileX + Lds<MT>::kXLo);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t w = j == 0 ? qm[t][b].x : j == 1 ? qm[t][b].y : j == 2 ? qm[t][b].z : qm[t][b].w;
                half8 bh, br;
                decode8<MT>(w, ch, bh, br);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    f32x16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mt], bh, j == 0 ? f32x16{} : cb[t][mt], 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[mt], bh, c, 0, 0, 0);
                    cb[t][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mt], br, c, 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sblk = b == 0 ? sc[t].x : b == 1 ? sc[t].y : b == 2 ? sc[t].z : sc[t].w;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[t][mt][r] = fmaf(sblk, cb[t][mt][r], acc[t][mt][r]);
        }
        // One block at a time: otherwise the scheduler hoists every block's
        // table reads and runs out of registers.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Wave w owns row tiles t < NT of the workgroup's row group (256*NT rows):
// rows group0 + 256t + 32w, against MT token tiles of 32 (tokens 32mt ..).
// A unit is (sub-slice i, tile t); ring slot (i*NT + t) % R holds it.
template <int NT, int MT>
__global__ __launch_bounds__(kMmThreads) void nf4_mm_kernel(MmArgs a) {
    // Ring of weight units in registers: four sub-slices ahead with one
    // row tile and one token tile, else two units ahead (the register
    // budget).
    constexpr int R = NT == 1 && MT == 1 ? 4 : 2;
    constexpr int SP = R / NT;                   // sub-slices per ring pass
    static_assert((NT == 1 || NT == 2) && (MT == 1 || MT == 2) && NT * MT <= 2, "tiles per wave");
    using L = Lds<MT>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: segment choice in scalar registers
    const int h = lane >> 5;
    const int nl = lane & 31;                    // this lane's token row (A) and weight row (B) in a tile
    const int slice = blockIdx.x;
    const int sub0 = slice * a.q;
    const int nsub = min(a.q, (a.K / kSub) - sub0);   // sub-slices of this slice (>= 1)
    const int kw0 = sub0 * kSub;                 // this workgroup's first K element
    const int group0 = blockIdx.y * (kGroupRows * NT);
    TileRef tr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) tr[t] = tile_ref(a, group0 + t * kGroupRows + wave * 32);
    const float *const x = a.x;
    const int M = a.M, K = a.K;

    // Activations one sub-slice ahead, weight units a ring pass ahead. Issue
    // order per sub-slice: activations, then its weight units; the prologue
    // issues in the same order so the loop's wait counts hold from its first
    // pass.
    // Loads past the slice's end (a ring refill beyond its last sub-slice)
    // are dummies of one line each, so every pass issues the same sequence
    // and the compiler's wait counts stay exact.
    const XBase<MT> xb = x_base<MT>(x, M, K, tid);
    UnitBase ub[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ub[t] = unit_base(tr[t], K, lane);
    f32x4 xr[4 * MT];
    Unit ring[R];
    load_x<MT>(xr, xb, kw0, true, x);
#pragma unroll
    for (int r = 0; r < R; ++r) issue_unit(ring[r], ub[r % NT], kw0 + (r / NT) * kSub, r / NT < nsub, tr[r % NT].w);
    build_table<MT>(tid);

    const uint32_t ch = MT == 1 ? nl * 4 : (nl & 15) * 8;
    uint32_t arow = L::kXOff + (nl * kRS + 32 * h) * 2;
    asm volatile("" : "+v"(arow));               // one base register: element offsets stay immediates
    const uint32_t cst = L::kCOff + wave * 32 * kCRow, sst = L::kSOff + wave * 32 * 16;
    f32x16 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][mt][r] = 0.0f;

    // Sub-slice i = p0 + PS: stage its activations between two barriers,
    // fetch i+1's, compute its NT units (ring slots PS*NT ..) and refill
    // those slots with the units of sub-slice i + SP. Past the slice's end
    // the loads are dummies and nothing is computed.
    auto step = [&](int p0, auto ps) {
        constexpr int PS = decltype(ps)::value;
        const int i = p0 + PS;
        if (i < nsub) {
            __syncthreads();                     // every wave is done with sub-slice i-1's activations
            stage_x<MT>(xr, tid);
            __syncthreads();                     // sub-slice i's activations (and the table) visible
        }
        load_x<MT>(xr, xb, kw0 + (i + 1) * kSub, i + 1 < nsub, x);
        if (i < nsub) compute_units<NT, MT>(acc, ring + PS * NT, arow, cst, sst, lane, ch);
#pragma unroll
        for (int t = 0; t < NT; ++t) issue_unit(ring[PS * NT + t], ub[t], kw0 + (i + SP) * kSub, i + SP < nsub, tr[t].w);
    };
    for (int p0 = 0; p0 < nsub; p0 += SP) {
        step(p0, std::integral_constant<int, 0>{});
        if constexpr (SP == 2) step(p0, std::integral_constant<int, 1>{});
        if constexpr (SP == 4) {
            step(p0, std::integral_constant<int, 1>{});
            step(p0, std::integral_constant<int, 2>{});
            step(p0, std::integral_constant<int, 3>{});
        }
    }

    // Accumulator r of token tile mt, lane l is C[token 32mt + 8*(r/4) +
    // 4*h + r%4][row nl].
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = tr[t].local0 + nl;
        if (n >= tr[t].n) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (a.part == nullptr) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < a.M) {
                        float *yp = tr[t].y + static_cast<size_t>(m) * tr[t].n + n;
                        *yp = a.add ? *yp + acc[t][mt][r] : acc[t][mt][r];
                    }
                }
            } else {
                float *const ps =
                    a.part + static_cast<size_t>(slice) * a.M * a.N + group0 + t * kGroupRows + wave * 32 + nl;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (m < a.M) ps[static_cast<size_t>(m) * a.N] = acc[t][mt][r];
                }
            }
        }
    }
}

// Y (+)= the slices' partial sums, added in slice order: thread per output
// element (m, stacked row n). Shared by the NF4 and K-quant GEMMs.
struct ReduceArgs {
    float *y[3];
    int end[3];
    int nseg;
    int M, N, slices, add;
    const float *part;
};

__global__ __launch_bounds__(256) void nf4_mm_reduce_kernel(ReduceArgs r) {
    const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<long long>(r.M) * r.N) return;
    const int m = static_cast<int>(idx / r.N), n = static_cast<int>(idx % r.N);
    const float v = slice_sum(r.part + idx, static_cast<size_t>(r.M) * r.N, r.slices);
    const int seg = segment_of(r.end, r.nseg, n);
    const int start = seg == 0 ? 0 : seg == 1 ? r.end[0] : r.end[1];
    const int sn = (seg == 0 ? r.end[0] : seg == 1 ? r.end[1] : r.end[2]) - start;
    float *yp = (seg == 0 ? r.y[0] : seg == 1 ? r.y[1] : r.y[2]) + static_cast<size_t>(m) * sn + (n - start);
    *yp = r.add ? *yp + v : v;
}

// ---------------------------------------------------------------------------
// NF4 GEMM with the activations held in registers (nf4_gemm_kernel), for
// K % 1024 == 0 and passes of up to 64 tokens.
//
// Precision: the activations are rounded to fp16 (to nearest; an A image
// built once per call by nf4_xpack_kernel, or written by the decode step's
// tail that produced them) and each NF4 level is exact as H + R (H = fp16 of
// the level, R = fp16 of the rest): one table entry per code byte holds both
// pairs, a B fragment is {H0 H1 R0 R1 H2 H3 R2 R3} of four weights and the A
// fragment repeats each activation pair against it, so every product is
// x16 * (H + R) accumulated in fp32. A token row is within the activations'
// rounding of the fp32 result (~2e-4 relative).
//
// Work split: slice s of K (blockIdx.x) spans 8 waves x KS = 64*NB
// elements; wave w owns [(8s + w)*KS, +KS) and keeps that range of all M
// token rows in registers as A fragments, loaded once. The workgroup walks
// 16-row tiles t = blockIdx.y + i*gridDim.y. Each wave streams its K range of
// the tiles' 16 weight rows (codes and absmax) into a private ring of D tile
// slots in LDS with LDS-DMA loads (no staging registers, so nothing in flight
// crosses the loop in registers), waits for the oldest slot with an explicit
// vmcnt, reads it into registers, refills it D tiles ahead, then decodes
// through the LDS table (the next dword's reads issued before the current
// dword's MFMAs), runs each 64-element block into fresh accumulators (two
// independent MFMA chains per token tile) and adds them scaled by the
// block's absmax. The 8 waves' 16 x M partial tiles are summed in wave order
// through LDS and written (or stored as the slice's partials for the
// slice-sum or tail kernel): deterministic, no atomics.
//
// v_mfma_f32_16x16x32_f16: lane l = 16g + i supplies A[i][8g + e] and
// B[8g + e][i] (e < 8); accumulator r of lane l is C[4g + r][i]. A is the
// activations (i = token), B the weights (i = weight row). K order: in block
// b (elements kw + 64b ..), lane group g covers elements 16g .. 16g+15 (the
// 8 code bytes 8g .. 8g+7 of the row's 32-byte block segment) in four MFMAs
// of four elements each, so each MFMA stays inside one absmax block.
//
// Slot image (per tile, per wave): NB/2 code windows of 1 KiB (window j =
// blocks 2j, 2j+1 of the 16 rows: DMA lane l loads row l%16, bytes
// 16*(l/16) .. +16 of the row's 64-byte window, landing at 16*l), then the
// 16 x NB absmax floats row-major. A lane's 8 code bytes of block b sit at
// 1024*(b/2) + 16*(16*(2*(b%2) + g/2) + i) + 8*(g%2): the 64 lanes of one
// block read 512 contiguous bytes.

typedef float f32x4m __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2m __attribute__((ext_vector_type(2)));
typedef u32x2m __attribute__((address_space(3))) lds_u32x2m;
typedef f32x4m __attribute__((address_space(3))) lds_f32x4m;

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = kGemmWaves * 64;
constexpr uint32_t kGemmTable = Lds<1>::kTableBytes;      // the pair table, 32 replicas
constexpr uint32_t kGemmLdsMax = 160 * 1024;
constexpr int kAFirstTiles = 8;                               // see nf4_gemm_kernel's prologue

template <int MT, int NB>
struct GemmLds {
    // Partial tiles [wave][mt][r][lane] floats, two buffers.
    static constexpr uint32_t kRedBuf = kGemmWaves * MT * 4 * 64 * 4;
    static constexpr uint32_t kRedOff = kGemmTable;
    static constexpr uint32_t kRingOff = kRedOff + 2 * kRedBuf;
    static constexpr uint32_t kCodeBytes = 512 * NB;                    // 16 rows x 32 bytes per block
    static constexpr uint32_t kSlot = kCodeBytes + 64 * NB;             // + 16 x NB absmax floats
    static constexpr int kD = static_cast<int>((kGemmLdsMax - kRingOff) / (kGemmWaves * kSlot));
    static constexpr int D = kD > 4 ? 4 : kD;                           // tiles in flight per wave
    static constexpr uint32_t kBytes = kRingOff + kGemmWaves * D * kSlot;
    static constexpr int kDma = NB / 2 + (NB + 3) / 4;                  // DMA instructions per tile
    static_assert(NB % 2 == 0 && D >= 2 && kBytes <= kGemmLdsMax, "LDS budget of a CU");
};

struct GemmArgs {
    const float *x;          // [M][K]
    const u32x4v *xp;        // the activations' fp16 fragment image (nf4_xpack_kernel)
    const uint8_t *w[3];
    const float *absmax[3];
    float *y[3];
    int end[3];              // stacked-row ends; every segment but the last a multiple of 16 rows
    int nseg;
    int M, N, K;
    int add;                 // Y += (one slice, no partial buffer)
    float *part;             // [slices][M][N] partial sums, or null: Y directly
    int tiles;               // ceil(N / 16)
};

struct GemmTile {
    const uint8_t *w;
    const float *absmax;
    float *y;
    int local0, n;
};

// Branch-free select of a uniform segment index s in {0, 1, 2}: masks and
// adds on scalar values, so neither a branch nor an indexed read of the
// argument block is formed.
template <typename T>
__device__ __forceinline__ T seg_pick(T v0, T v1, T v2, int s) {
    const uint64_t a0 = (uint64_t)v0, a1 = (uint64_t)v1, a2 = (uint64_t)v2;
    const uint64_t m1 = 0 - static_cast<uint64_t>(s >= 1), m2 = 0 - static_cast<uint64_t>(s >= 2);
    return (T)(a0 + ((a1 - a0) & m1) + ((a2 - a1) & m2));
}

__device__ __forceinline__ GemmTile gemm_tile(const GemmArgs &a, int r0) {
    const int e0 = a.end[0], e1 = a.end[1], e2 = a.end[2];
    int s = (r0 >= e0) + (r0 >= e1);
    s = s > a.nseg - 1 ? a.nseg - 1 : s;
    GemmTile t;
    t.w = seg_pick(a.w[0], a.w[1], a.w[2], s);
    t.absmax = seg_pick(a.absmax[0], a.absmax[1], a.absmax[2], s);
    t.y = seg_pick(a.y[0], a.y[1], a.y[2], s);
    const int start = seg_pick(0, e0, e1, s);
    t.local0 = r0 - start;
    t.n = seg_pick(e0, e1, e2, s) - start;
    return t;
}

// s_waitcnt with only the vector-memory count limited (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Waits until at most min(n, J) tiles of KD vector-memory loads each are
// still in flight (n uniform): the tiles issued after the awaited one, fewer
// than the ring depth near the end of a workgroup's walk, where no load is
// issued past its last tile.
template <int KD, int J>
__device__ __forceinline__ void wait_tiles(int n) {
    if constexpr (J == 0) {
        wait_vmcnt<0>();
    } else {
        if (n >= J)
            wait_vmcnt<J * KD>();
        else
            wait_tiles<KD, J - 1>(n);
    }
}

// LDS-DMA loads (global_load_lds: 16 or 4 bytes per lane, landing at
// `lds_base` + size * lane). Written as inline assembly: the compiler models
// the builtin like a FLAT access that also counts on the LDS counter and
// then waits for every outstanding LDS read before using any of them, which
// would serialize the table lookups; the hardware counts these loads on the
// vector-memory counter only, and every wait for their data here is an
// explicit vmcnt. M0 carries the LDS address (latched at issue, one wait
// state after it is written) and is restored afterwards.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds_base) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(lds_base), "v"(g)
                 : "memory");
}
__device__ __forceinline__ void dma4(const void *g, uint32_t lds_base) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %2, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(save)
                 : "s"(lds_base), "v"(g)
                 : "memory");
}

// LDS-DMA loads of one tile (this wave's K range of rows 16t .. 16t+15) into
// the slot at LDS byte `slot` (uniform): NB/2 16-byte code loads per lane,
// then the absmax floats (4 bytes per lane; lanes past 16*NB floats idle).
template <int NB>
__device__ __forceinline__ void gemm_dma(const GemmArgs &a, int tile, int kw, uint32_t slot, int lane) {
    const GemmTile tr = gemm_tile(a, tile * 16);
    const int crow = min(tr.local0 + (lane & 15), tr.n - 1);
    const uint8_t *qp = tr.w + static_cast<size_t>(crow) * (a.K >> 1) + (kw >> 1) + 16 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < NB / 2; ++j) dma16(qp + 64 * j, slot + 1024 * j);
#pragma unroll
    for (int j = 0; j < (NB + 3) / 4; ++j) {
        const int f = lane + 64 * j;             // float f of the tile image: row f / NB, block f % NB
        const int srow = min(tr.local0 + f / NB, tr.n - 1);
        const float *sp = tr.absmax + static_cast<size_t>(srow) * (a.K >> 6) + (kw >> 6) + f % NB;
        if (16 * NB % 64 == 0 || f < 16 * NB) dma4(sp, slot + 512 * NB + 256 * j);
    }
}

// The activation-stationary GEMM's decode table: 256 entries (a code byte:
// the even element in the high nibble) of 8 bytes, the byte's fp16 level
// pair {H(e >> 4), H(e & 15)} and residual pair {R(e >> 4), R(e & 15)}
// (H = the level rounded to nearest fp16, R = fp16(level - H); H + R is the
// fp32 level to within 2^-22 of it), in 32 replicas: entry e, replica r at
// e*256 + 8r. Thread tid (of 512) fills replica tid % 32 of entries
// e0 + 16j (e0 = tid / 32 < 16, j < 16): the high nibble j is a constant of
// the unrolled loop, the low nibble e0.
__device__ __forceinline__ void build_table_hr(int tid) {
    constexpr float kNF4[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
    const uint32_t r = static_cast<uint32_t>(tid & 31) * 8;
    const int e0 = tid >> 5;
    const float lo = nf4_level_sel(e0);
    const float lo_r = level_rest(lo);
#pragma unroll
    for (int j = 0; j < 16; ++j)
        *lds<lds_u32x2m>(static_cast<uint32_t>(16 * j + e0) * 256 + r) =
            u32x2m{pack_half2(kNF4[j], lo), pack_half2(level_rest(kNF4[j]), lo_r)};
}

// B fragments of code dword `w` through build_table_hr: byte t's entry
// (address: one v_perm of the byte into bits 8..15 beside ch = 8 * (lane %
// 32)) lands as {H pair, R pair}; bytes 0, 1 form the first fragment
// (K slots H0 H1 R0 R1 H2 H3 R2 R3 of the dword's elements 0..3), bytes 2, 3
// the second (elements 4..7).
__device__ __forceinline__ void decode8_hr(uint32_t w, uint32_t ch, half8 &f0, half8 &f1) {
    const u32x2m e0 = *lds<lds_u32x2m>(__builtin_amdgcn_perm(w, ch, 0x0C0C0400u));
    const u32x2m e1 = *lds<lds_u32x2m>(__builtin_amdgcn_perm(w, ch, 0x0C0C0500u));
    const u32x2m e2 = *lds<lds_u32x2m>(__builtin_amdgcn_perm(w, ch, 0x0C0C0600u));
    const u32x2m e3 = *lds<lds_u32x2m>(__builtin_amdgcn_perm(w, ch, 0x0C0C0700u));
    f0 = __builtin_bit_cast(half8, u32x4v{e0.x, e0.y, e1.x, e1.y});
    f1 = __builtin_bit_cast(half8, u32x4v{e2.x, e2.y, e3.x, e3.y});
}

// The activations as the GEMM's A operand, once per call: fp16 (rounded to
// nearest) in the order the fragments need, [mt][64-element block kb][jj]
// [lane] as 8 fp16 per entry: lane l = 16g + i holds token 16mt + i (zero
// past M), elements 64kb + 16g + 8jj .. +8. A wave of the GEMM loads each
// piece as 1 KiB contiguous and duplicates each element pair in registers
// (the K slots x0 x1 x0 x1 x2 x3 x2 x3 that meet H0 H1 R0 R1 H2 H3 R2 R3).
__global__ __launch_bounds__(256) void nf4_xpack_kernel(const float *x, u32x4v *xp, int M, int K, int total) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int lane = idx & 63, jj = (idx >> 6) & 1, kbs = K >> 6;
    const int kb = (idx >> 7) % kbs, mt = (idx >> 7) / kbs;
    const int m = 16 * mt + (lane & 15);
    f32x4m lo4 = {0.0f, 0.0f, 0.0f, 0.0f}, hi4 = lo4;
    if (m < M) {
        const float *src = x + static_cast<size_t>(m) * K + 64 * kb + 16 * (lane >> 4) + 8 * jj;
        lo4 = gload<f32x4m>(src);
        hi4 = gload<f32x4m>(src + 4);
    }
    xp[(static_cast<size_t>(mt * kbs + kb) * 2 + jj) * 64 + lane] =
        u32x4v{pack_half2(lo4.x, lo4.y), pack_half2(lo4.z, lo4.w), pack_half2(hi4.x, hi4.y), pack_half2(hi4.z, hi4.w)};
}

// A 16-byte global load whose completion the compiler does not track: the
// caller waits for it with an explicit vmcnt and passes the value through
// settle() before any use.
__device__ __forceinline__ u32x4v gload_untracked(const u32x4v *p) {
    u32x4v v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
// After the explicit wait: ties the loaded registers to this point, so no
// instruction reads them earlier.
__device__ __forceinline__ void settle(u32x4v &v) { asm volatile("" : "+v"(v)); }

// The tile's 16 x MT*16 partial sums of the 8 waves through LDS at `rb`,
// summed in wave order and written to the slice partials or the outputs.
// Lane l of wave w stored accumulator mt at ((w*MT + mt)*64 + l)*16.
template <int MT>
__device__ __forceinline__ void gemm_tile_out(const GemmArgs &a, uint32_t rb, int tile, int tid) {
    const GemmTile tr = gemm_tile(a, tile * 16);
#pragma unroll
    for (int o0 = 0; o0 < 256 * MT; o0 += kGemmThreads) {
        const int o = o0 + tid;
        if (256 * MT % kGemmThreads != 0 && o >= 256 * MT) break;
        const int mt = o >> 8, lq = (o >> 2) & 63, r = o & 3;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kGemmWaves; ++w) v += __uint_as_float(*lds<lds_u32>(rb + (w * MT * 64 * 4 + o) * 4));
        const int token = 16 * mt + 4 * (lq >> 4) + r, n = lq & 15, local = tr.local0 + n;
        if (token < a.M && local < tr.n) {
            typedef float __attribute__((address_space(1))) gf32;
            if (a.part != nullptr) {
                *(gf32 *)(a.part + (static_cast<size_t>(blockIdx.x) * a.M + token) * a.N + tile * 16 + n) = v;
            } else {
                gf32 *yp = (gf32 *)(tr.y + static_cast<size_t>(token) * tr.n + local);
                *yp = a.add ? *yp + v : v;
            }
        }
    }
}

// RT == 0: the waves' partial tiles meet in LDS after every tile (two
// buffers, one barrier per tile). RT > 0 (the host guarantees that a
// workgroup walks at most RT tiles): each wave keeps its partial tiles in
// registers and they meet once, after the last tile, in the LDS the table and
// the ring no longer need; the waves then run the whole loop without a
// barrier.
template <int MT, int NB, int RT>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(GemmArgs a) {
    constexpr int KS = 64 * NB;
    using GL = GemmLds<MT, NB>;
    constexpr int D = GL::D;
    static_assert(RT == 0 || RT * kGemmWaves * MT * 1024 <= GL::kBytes, "final reduction fits the LDS");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const int kw = (static_cast<int>(blockIdx.x) * kGemmWaves + wave) * KS;
    const int stride = gridDim.y;
    const int last = a.tiles - 1;
    const uint32_t ring = GL::kRingOff + wave * D * GL::kSlot;

    // The wave's A fragments first (16-byte loads of the fragment image,
    // 1 KiB contiguous per instruction; block b of token tile mt as two
    // pieces), then the first D tiles' weight loads. On a short walk (at most
    // kAFirstTiles tiles) the fragments land before any weight load is
    // issued, so they do not queue behind the chip-wide flood of ring loads
    // and the first tile starts earlier; a longer walk gains more from having
    // its first tiles in flight during that wait (measured on the decode
    // step's Wo, Q/K/V, down and gate/up walks of 2, 3, 8 and 14 tiles).
    int tile = blockIdx.y;
    int left = (last - tile) / stride;           // tiles of the walk after the current one
    const int kbs = a.K >> 6;
    u32x4v raw[MT][NB][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                raw[mt][b][jj] = gload_untracked(a.xp + (static_cast<size_t>(mt * kbs + (kw >> 6) + b) * 2 + jj) * 64 + lane);
    if (left < kAFirstTiles) {
        build_table_hr(tid);
        wait_vmcnt<0>();                         // the A fragment loads have landed
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (d <= left) gemm_dma<NB>(a, tile + d * stride, kw, ring + d * GL::kSlot, lane);
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d) gemm_dma<NB>(a, tile + d * stride, kw, ring + d * GL::kSlot, lane);
        build_table_hr(tid);
        wait_vmcnt<D * GL::kDma>();              // the A fragment loads (issued first) have landed
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) settle(raw[mt][b][jj]);
    // Element pairs duplicated: x0 x1 x0 x1 x2 x3 x2 x3 against H0 H1 R0 R1
    // H2 H3 R2 R3.
    half8 ax[MT][NB][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const u32x4v v = raw[mt][b][jj];
                ax[mt][b][2 * jj] = __builtin_bit_cast(half8, u32x4v{v.x, v.x, v.y, v.y});
                ax[mt][b][2 * jj + 1] = __builtin_bit_cast(half8, u32x4v{v.z, v.z, v.w, v.w});
            }
    lds_barrier();                               // the table

    const uint32_t ch = static_cast<uint32_t>(lane & 31) * 8;
    // Lane's code offset within a slot for block 0 (block b adds
    // 1024*(b/2) + 512*(b%2)) and its row's absmax offset.
    const uint32_t coff = 16 * (16 * (g >> 1) + i16) + 8 * (g & 1);
    const uint32_t soff = GL::kCodeBytes + 4 * NB * i16;
    int slot = 0;
    int buf = 0;
    f32x4m keep[RT > 0 ? RT : 1][MT];
    int nt = 0;
    for (;;) {
        const uint32_t sb = ring + slot * GL::kSlot;
        wait_tiles<GL::kDma, D - 1>(left);       // this tile's DMA loads have landed
        u32x2m q[NB];
        float sc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) q[b] = *lds<lds_u32x2m>(sb + coff + 1024 * (b >> 1) + 512 * (b & 1));
#pragma unroll
        for (int b = 0; b < NB; b += 4) {
            if (b + 4 <= NB) {
                const f32x4m v = *lds<lds_f32x4m>(sb + soff + 4 * b);
                sc[b] = v.x; sc[b + 1] = v.y; sc[b + 2] = v.z; sc[b + 3] = v.w;
            } else {
                const f32x2 v = *lds<lds_f32x2>(sb + soff + 4 * b);
                sc[b] = v.x; sc[b + 1] = v.y;
            }
        }
        wait_lgkmcnt0();                         // the slot is read: refill it D tiles ahead
        if (left >= D) gemm_dma<NB>(a, tile + D * stride, kw, sb, lane);

        // Per block b: dwords 2b (.x) and 2b+1 (.y) of the codes, each decoded
        // by four table reads into two B fragments; the reads of dword d+2
        // go out before the MFMAs of dword d (at most 12 reads outstanding:
        // the LDS counter tracks 15). The block's four MFMAs form one chain
        // per token tile (two buffers, by block parity), scaled into acc one
        // block later.
        f32x4m acc[MT], f[2][MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4m{0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4m z4 = {0.0f, 0.0f, 0.0f, 0.0f};
        half8 hb[4][2];
        decode8_hr(q[0].x, ch, hb[0][0], hb[0][1]);
        decode8_hr(q[0].y, ch, hb[1][0], hb[1][1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int cb = (2 * b) & 3;
            f32x4m (&fc)[MT] = f[b & 1];
            if (b + 1 < NB) decode8_hr(q[b + 1].x, ch, hb[(cb + 2) & 3][0], hb[(cb + 2) & 3][1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                fc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[mt][b][0], hb[cb][0], z4, 0, 0, 0);
                fc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[mt][b][1], hb[cb][1], fc[mt], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (b + 1 < NB) decode8_hr(q[b + 1].y, ch, hb[(cb + 3) & 3][0], hb[(cb + 3) & 3][1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                fc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[mt][b][2], hb[cb + 1][0], fc[mt], 0, 0, 0);
                fc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[mt][b][3], hb[cb + 1][1], fc[mt], 0, 0, 0);
            }
            // The previous block's products are ready by now: scale them in.
            if (b > 0) {
                const f32x4m (&fp)[MT] = f[(b - 1) & 1];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc[mt].x = fmaf(sc[b - 1], fp[mt].x, acc[mt].x);
                    acc[mt].y = fmaf(sc[b - 1], fp[mt].y, acc[mt].y);
                    acc[mt].z = fmaf(sc[b - 1], fp[mt].z, acc[mt].z);
                    acc[mt].w = fmaf(sc[b - 1], fp[mt].w, acc[mt].w);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const f32x4m fl = f[(NB - 1) & 1][mt];
            acc[mt].x = fmaf(sc[NB - 1], fl.x, acc[mt].x);
            acc[mt].y = fmaf(sc[NB - 1], fl.y, acc[mt].y);
            acc[mt].z = fmaf(sc[NB - 1], fl.z, acc[mt].z);
            acc[mt].w = fmaf(sc[NB - 1], fl.w, acc[mt].w);
        }

        if constexpr (RT > 0) {
            // Kept in registers (the index is uniform and unrolled).
#pragma unroll
            for (int t = 0; t < RT; ++t)
                if (t == nt)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) keep[t][mt] = acc[mt];
            ++nt;
        } else {
            // The waves' partial tiles through LDS, summed in wave order:
            // lane l of wave w stores its 4 accumulators of token tile mt as
            // one 16-byte piece at ((w*MT + mt)*64 + l)*16; thread o reads
            // piece o/4, element o%4 of every wave (consecutive threads,
            // consecutive addresses).
            const uint32_t rb = GL::kRedOff + buf * GL::kRedBuf;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) *lds<lds_f32x4m>(rb + ((wave * MT + mt) * 64 + lane) * 16) = acc[mt];
            lds_barrier();
            gemm_tile_out<MT>(a, rb, tile, tid);
        }
        buf ^= 1;
        slot = slot + 1 == D ? 0 : slot + 1;
        tile += stride;
        if (--left < 0) break;
    }
    wait_vmcnt<0>();                             // no LDS-DMA write may land after the wave ends (or in the reduction)
    if constexpr (RT > 0) {
        // Every wave is past its last table read and ring slot: the whole
        // LDS holds tile t's partials at t * 8 * MT KiB.
        lds_barrier();
#pragma unroll
        for (int t = 0; t < RT; ++t)
            if (t < nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    *lds<lds_f32x4m>(t * (kGemmWaves * MT * 1024) + ((wave * MT + mt) * 64 + lane) * 16) = keep[t][mt];
        lds_barrier();
        for (int t = 0; t < nt; ++t)
            gemm_tile_out<MT>(a, t * (kGemmWaves * MT * 1024), blockIdx.y + t * stride, tid);
    }
}

// ---- GGUF Q4_0 / Q8_0 GEMM with the activations held in registers -------
//
// The NF4 GEMM's structure for the 32-element GGUF blocks (18-byte Q4_0 {fp16
// d, 16 code bytes}, 34-byte Q8_0 {fp16 d, 32 int8}), passes of up to 16
// tokens: wave w of K slice s owns the elements [(8s + w)*KB, +KB) (KB = 32 *
// NBK, NBK a multiple of 8 so that a row's share starts 16-byte aligned) and
// keeps that range of the 16 token rows as fp16 hi and lo A fragments (x = hi
// + lo to 2^-22); each 16-row tile's share of the weights (16 rows x NBK
// blocks) streams into the wave's LDS ring by LDS-DMA, one MFMA pair per
// block (hi, then lo, against the same B) into a fresh 16 x 16 tile that the
// block's d scales into the accumulators. B holds the block's codes as exact
// fp16 integers (Q4_0: q - 8; Q8_0: q), built from the code bytes with v_perm
// against a constant 0x64 byte and one packed fp16 add (no table), so the
// result is the fp32 matvec to ~2^-22 per product. Partial tiles meet across
// the waves as in the NF4 kernel.
//
// MFMA 16x16x32 per block: lane l = 16g + i supplies A[i][8g + e] (token i,
// block elements 8g..8g+7) and B[8g + e][i] (row i). Q4_0 elements 0..15 are
// the low nibbles of code bytes 0..15 and 16..31 the high nibbles, so lane
// group g reads code bytes 8(g & 1) .. +7 and takes nibble g >> 1; Q8_0 lane
// group g reads bytes 8g .. 8g+7.
//
// Slot image: the DMA instruction j, lane l loads 16-byte piece 4j + l/16 of
// row l % 16's share, landing at 1024j + 16l: byte c of row r sits at
// 256*(c/16) + 16r + c%16 (lanes past the share re-read its last piece into
// the slot's tail).

template <int F> struct GgFmt {                  // F: 0 = Q4_0, 1 = Q8_0
    static constexpr int BB = F == 0 ? 18 : 34;
};

template <int F, int NBK>
struct GgLds {
    static constexpr int RB = NBK * GgFmt<F>::BB;                        // a row's share, bytes
    static constexpr int PR = RB / 16;                                   // its 16-byte pieces
    static constexpr int kDma = (PR + 3) / 4;                            // DMA instructions per tile
    static constexpr uint32_t kSlot = kDma * 1024;
    static constexpr uint32_t kRedBuf = kGemmWaves * 4 * 64 * 4;         // one token tile
    static constexpr uint32_t kRedOff = 0;
    static constexpr uint32_t kRingOff = 2 * kRedBuf;
    static constexpr int kD = static_cast<int>((kGemmLdsMax - kRingOff) / (kGemmWaves * kSlot));
    static constexpr int D = kD > 4 ? 4 : kD;
    static constexpr uint32_t kBytes = kRingOff + kGemmWaves * D * kSlot;
    static_assert(RB % 16 == 0 && D >= 2 && kBytes <= kGemmLdsMax, "ring of at least two tiles");
};

template <int F, int NBK>
__device__ __forceinline__ void gg_dma(const GemmArgs &a, int tile, int kw, uint32_t slot, int lane) {
    using GL = GgLds<F, NBK>;
    const GemmTile tr = gemm_tile(a, tile * 16);
    const int crow = min(tr.local0 + (lane & 15), tr.n - 1);
    const uint8_t *rp = tr.w + static_cast<size_t>(crow) * (static_cast<size_t>(a.K >> 5) * GgFmt<F>::BB) +
                        static_cast<size_t>(kw >> 5) * GgFmt<F>::BB;
#pragma unroll
    for (int j = 0; j < GL::kDma; ++j) {
        const int p = 4 * j + (lane >> 4);
        dma16(rp + 16 * (p < GL::PR ? p : GL::PR - 1), slot + 1024 * j);
    }
}

// Dword of row r's share at byte c (c % 4 == 0) in the slot image.
__device__ __forceinline__ uint32_t gg_word(uint32_t sb, int r, int c) {
    return *lds<lds_u32>(sb + 256 * (c >> 4) + 16 * r + (c & 15));
}

// Halves 0x64bb of bytes 2t and 2t+1 of `w` (v_perm against a constant
// 0x64 byte): 1024 + byte, exact.
template <int T>
__device__ __forceinline__ uint32_t gg_magic(uint32_t w) {
    return __builtin_amdgcn_perm(0x64646464u, w, 0x04000400u | ((2u * T + 1u) << 16) | (2u * T));
}
__device__ __forceinline__ uint32_t gg_hadd(uint32_t v, uint32_t c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v) + __builtin_bit_cast(h2, c));
}

template <int F, int NBK, int RT>
__global__ __launch_bounds__(kGemmThreads) void gguf_gemm_kernel(GemmArgs a) {
    constexpr int KB = 32 * NBK;
    using GL = GgLds<F, NBK>;
    constexpr int D = GL::D;
    constexpr int BB = GgFmt<F>::BB;
    static_assert(RT == 0 || RT * kGemmWaves * 1024 <= GL::kBytes, "final reduction fits the LDS");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const int kw = (static_cast<int>(blockIdx.x) * kGemmWaves + wave) * KB;
    const int stride = gridDim.y;
    const int last = a.tiles - 1;
    const uint32_t ring = GL::kRingOff + wave * D * GL::kSlot;

    // The activations first (token i16, block elements 8g .. 8g+7 of each
    // block: two 16-byte loads per block; lanes of rows past M load nothing
    // and hold zeros), then the first D tiles' weights.
    int tile = blockIdx.y;
    int left = (last - tile) / stride;           // tiles of the walk after the current one
    const bool live = i16 < a.M;
    const float *xr = a.x + static_cast<size_t>(live ? i16 : 0) * a.K + kw + 8 * g;
    u32x4v raw[NBK][2];
#pragma unroll
    for (int b = 0; b < NBK; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) raw[b][h] = u32x4v{0u, 0u, 0u, 0u};
    if (live) {
#pragma unroll
        for (int b = 0; b < NBK; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) raw[b][h] = gload_untracked(reinterpret_cast<const u32x4v *>(xr + 32 * b + 4 * h));
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d <= left) gg_dma<F, NBK>(a, tile + d * stride, kw, ring + d * GL::kSlot, lane);
    wait_tiles<GL::kDma, D>(left + 1);           // the activation loads (issued first) have landed
#pragma unroll
    for (int b = 0; b < NBK; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) settle(raw[b][h]);
    half8 ah[NBK], al[NBK];
#pragma unroll
    for (int b = 0; b < NBK; ++b) {
        float v[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v[4 * h + 0] = __uint_as_float(raw[b][h].x);
            v[4 * h + 1] = __uint_as_float(raw[b][h].y);
            v[4 * h + 2] = __uint_as_float(raw[b][h].z);
            v[4 * h + 3] = __uint_as_float(raw[b][h].w);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const _Float16 hi = static_cast<_Float16>(v[e]);
            ah[b][e] = hi;
            al[b][e] = static_cast<_Float16>(v[e] - static_cast<float>(hi));
        }
    }

    // Q4_0: nibble g >> 1 of code bytes 8(g & 1) ..; Q8_0: bytes 8g ..
    const int cg = F == 0 ? 8 * (g & 1) : 8 * g;
    const uint32_t nsh = F == 0 ? 4u * static_cast<uint32_t>(g >> 1) : 0u;
    const uint32_t bias = F == 0 ? 0xE408E408u : 0xE480E480u;   // fp16 -1032 (Q4_0) / -1152 (Q8_0) pairs
    int slot = 0;
    int buf = 0;
    f32x4m keep[RT > 0 ? RT : 1];
    int nt = 0;
    for (;;) {
        const uint32_t sb = ring + slot * GL::kSlot;
        wait_tiles<GL::kDma, D - 1>(left);       // this tile's DMA loads have landed
        // The tile's code words and scales into registers, then the slot is
        // refilled D tiles ahead.
        uint32_t cw[NBK][2];
        float dsc[NBK];
#pragma unroll
        for (int b = 0; b < NBK; ++b) {
            const int c = BB * b + 2 + cg;       // c % 4 is (2b + 2) % 4 for both formats
            if (((2 * b + 2) & 3) == 0) {
                cw[b][0] = gg_word(sb, i16, c);
                cw[b][1] = gg_word(sb, i16, c + 4);
            } else {
                const uint32_t w0 = gg_word(sb, i16, c - 2), w1 = gg_word(sb, i16, c + 2),
                               w2 = gg_word(sb, i16, c + 6);
                cw[b][0] = __builtin_amdgcn_alignbyte(w1, w0, 2);
                cw[b][1] = __builtin_amdgcn_alignbyte(w2, w1, 2);
            }
            const uint32_t dw = gg_word(sb, i16, (BB * b) & ~3);
            dsc[b] = f16_bits_to_f32((BB * b) & 2 ? dw >> 16 : dw & 0xffffu);
        }
        wait_lgkmcnt0();
        if (left >= D) gg_dma<F, NBK>(a, tile + D * stride, kw, sb, lane);

        f32x4m acc = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4m z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < NBK; ++b) {
            uint32_t w0 = cw[b][0], w1 = cw[b][1];
            if constexpr (F == 0) {
                w0 = (w0 >> nsh) & 0x0f0f0f0fu;
                w1 = (w1 >> nsh) & 0x0f0f0f0fu;
            } else {
                w0 ^= 0x80808080u;
                w1 ^= 0x80808080u;
            }
            const u32x4v bq = {gg_hadd(gg_magic<0>(w0), bias), gg_hadd(gg_magic<1>(w0), bias),
                               gg_hadd(gg_magic<0>(w1), bias), gg_hadd(gg_magic<1>(w1), bias)};
            const half8 bf = __builtin_bit_cast(half8, bq);
            f32x4m c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[b], bf, z4, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[b], bf, c, 0, 0, 0);
            acc.x = fmaf(dsc[b], c.x, acc.x);
            acc.y = fmaf(dsc[b], c.y, acc.y);
            acc.z = fmaf(dsc[b], c.z, acc.z);
            acc.w = fmaf(dsc[b], c.w, acc.w);
        }

        if constexpr (RT > 0) {
#pragma unroll
            for (int t = 0; t < RT; ++t)
                if (t == nt) keep[t] = acc;
            ++nt;
        } else {
            const uint32_t rb = GL::kRedOff + buf * GL::kRedBuf;
            *lds<lds_f32x4m>(rb + (wave * 64 + lane) * 16) = acc;
            lds_barrier();
            gemm_tile_out<1>(a, rb, tile, tid);
        }
        buf ^= 1;
        slot = slot + 1 == D ? 0 : slot + 1;
        tile += stride;
        if (--left < 0) break;
    }
    wait_vmcnt<0>();                             // no LDS-DMA write may land after the wave ends (or in the reduction)
    if constexpr (RT > 0) {
        lds_barrier();
#pragma unroll
        for (int t = 0; t < RT; ++t)
            if (t < nt) *lds<lds_f32x4m>(t * (kGemmWaves * 1024) + (wave * 64 + lane) * 16) = keep[t];
        lds_barrier();
        for (int t = 0; t < nt; ++t) gemm_tile_out<1>(a, t * (kGemmWaves * 1024), blockIdx.y + t * stride, tid);
    }
}

// ---- GGUF Q4_K GEMM with the activations held in registers --------------
//
// The NF4 GEMM's structure (the same fp16 A-fragment image, the same
// rounding of the activations to fp16 once) for Q4_K super-blocks: wave w of
// K slice s owns super-block 8s + w of every row (256 elements, 144 bytes:
// f16 d, f16 dmin, 12 bytes of 6-bit scale and min codes, qs[128] with
// elements 64c + l and 64c + 32 + l in the low and high nibble of byte
// 32c + l). A 64-element block c of the image holds, for lane l = 16g + i,
// elements 64c + 16g + 8jj + e (jj < 2, e < 8) of token i: the low nibbles of
// bytes 32c + 16(g%2) + 8jj + e when g < 2 (sub-block 2c), the high ones when
// g >= 2 (sub-block 2c + 1). B fragments are exact fp16 integers with the
// scale folded in, q*sc (<= 15*63 = 945: one packed fp16 FMA of the magic
// 1024 + q, exact), and a second pair of MFMAs against the min code m (<= 63)
// gives sum(x*m); the accumulators take d * (the first) - dmin * (the
// second), the min term only where one of the block's two min codes is
// non-zero (a zero min code adds nothing whatever dmin holds). The rows'
// shares of a tile (16 x 144 bytes) arrive by LDS-DMA exactly as the Q4_0
// ones with 8 blocks (the same slot image).
__device__ __forceinline__ uint32_t gg_hfma(uint32_t v, uint32_t s, uint32_t c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, v), __builtin_bit_cast(h2, s),
                                                                  __builtin_bit_cast(h2, c)));
}

// LDS of the Q4_K GEMM: the per-tile reduction buffers of MT token tiles,
// then the per-wave rings of NSB * 144-byte row shares (the Q4_0 slot of
// 8 * NSB blocks).
template <int MT, int NSB>
struct Q4kLds {
    static constexpr int kDma = GgLds<0, 8 * NSB>::kDma;
    static constexpr uint32_t kSlot = GgLds<0, 8 * NSB>::kSlot;
    static constexpr uint32_t kRedBuf = kGemmWaves * MT * 1024;
    static constexpr uint32_t kRedOff = 0;
    static constexpr uint32_t kRingOff = 2 * kRedBuf;
    static constexpr int kD = static_cast<int>((kGemmLdsMax - kRingOff) / (kGemmWaves * kSlot));
    static constexpr int D = kD > 4 ? 4 : kD;
    static constexpr uint32_t kBytes = kRingOff + kGemmWaves * D * kSlot;
    static_assert(D >= 2 && kBytes <= kGemmLdsMax, "ring of at least two tiles");
};

// The 6-bit scale and min codes of sub-blocks 2c and 2c+1 from the scale
// words w1 = bytes 4..7, w2 = 8..11, w3 = 12..15 of a Q4_K super-block.
__device__ __forceinline__ void q4k_codes6(uint32_t w1, uint32_t w2, uint32_t w3, int c, uint32_t &sc0,
                                           uint32_t &sc1, uint32_t &mn0, uint32_t &mn1) {
    const uint32_t o = 16 * (c & 1);
    if (c < 2) {
        sc0 = __builtin_amdgcn_ubfe(w1, o, 6);
        sc1 = __builtin_amdgcn_ubfe(w1, o + 8, 6);
        mn0 = __builtin_amdgcn_ubfe(w2, o, 6);
        mn1 = __builtin_amdgcn_ubfe(w2, o + 8, 6);
    } else {
        sc0 = __builtin_amdgcn_ubfe(w3, o, 4) | (__builtin_amdgcn_ubfe(w1, o + 6, 2) << 4);
        sc1 = __builtin_amdgcn_ubfe(w3, o + 8, 4) | (__builtin_amdgcn_ubfe(w1, o + 14, 2) << 4);
        mn0 = __builtin_amdgcn_ubfe(w3, o + 4, 4) | (__builtin_amdgcn_ubfe(w2, o + 6, 2) << 4);
        mn1 = __builtin_amdgcn_ubfe(w3, o + 12, 4) | (__builtin_amdgcn_ubfe(w2, o + 14, 2) << 4);
    }
}

template <int MT, int NSB, int RT>
__global__ __launch_bounds__(kGemmThreads) void q4k_gemm_kernel(GemmArgs a) {
    using GL = Q4kLds<MT, NSB>;
    constexpr int D = GL::D;
    static_assert(RT == 0 || RT * kGemmWaves * MT * 1024 <= GL::kBytes, "final reduction fits the LDS");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const int kw = (static_cast<int>(blockIdx.x) * kGemmWaves + wave) * 256 * NSB;
    const int stride = gridDim.y;
    const int last = a.tiles - 1;
    const uint32_t ring = GL::kRingOff + wave * D * GL::kSlot;
    constexpr int NC = 4 * NSB;                  // 64-element blocks per wave

    // The A fragments first (NC 64-element blocks per token tile, two
    // 16-byte loads each), then the first D tiles' weights.
    int tile = blockIdx.y;
    int left = (last - tile) / stride;           // tiles of the walk after the current one
    const int kbs = a.K >> 6;
    u32x4v raw[MT][NC][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
                raw[mt][c][jj] = gload_untracked(a.xp + (static_cast<size_t>(mt * kbs + (kw >> 6) + c) * 2 + jj) * 64 + lane);
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (d <= left) gg_dma<0, 8 * NSB>(a, tile + d * stride, kw, ring + d * GL::kSlot, lane);
    wait_tiles<GL::kDma, D>(left + 1);           // the fragment loads (issued first) have landed
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) settle(raw[mt][c][jj]);

    const uint32_t nsh = 4u * static_cast<uint32_t>(g >> 1);
    int slot = 0;
    int buf = 0;
    f32x4m keep[RT > 0 ? RT : 1][MT];
    int nt = 0;
    for (;;) {
        const uint32_t sb = ring + slot * GL::kSlot;
        wait_tiles<GL::kDma, D - 1>(left);       // this tile's DMA loads have landed
        // Row i16's header of each super-block (bytes 144u .. 144u+15: d,
        // dmin, the scale codes; 16-byte piece 9u) and its 16 code bytes of
        // each pair (bytes 144u + 16 + 32c + 16(g%2) ..), then the slot is
        // refilled D tiles ahead.
        u32x4v hdr[NSB];
        u32x4v qw[NC];
#pragma unroll
        for (int u = 0; u < NSB; ++u) {
            hdr[u] = *lds<lds_u32x4>(sb + 256 * (9 * u) + 16 * i16);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                qw[4 * u + c] = *lds<lds_u32x4>(sb + 256 * (9 * u + 1 + 2 * c + (g & 1)) + 16 * i16);
        }
        wait_lgkmcnt0();
        if (left >= D) gg_dma<0, 8 * NSB>(a, tile + D * stride, kw, sb, lane);

        f32x4m acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4m{0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4m z4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
            const int u = cc >> 2, c = cc & 3;
            const float dd = f16_bits_to_f32(hdr[u].x & 0xffffu);
            const float dmin = f16_bits_to_f32(hdr[u].x >> 16);
            uint32_t sc0, sc1, mn0, mn1;
            q4k_codes6(hdr[u].y, hdr[u].z, hdr[u].w, c, sc0, sc1, mn0, mn1);
            const uint32_t sc = g < 2 ? sc0 : sc1, mn = g < 2 ? mn0 : mn1;
            // fp16 pairs: sc (exact), -1024*sc (exact), mn (exact).
            const uint32_t sch = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(static_cast<float>(sc))));
            const uint32_t sc2 = sch | (sch << 16);
            const uint32_t nbh = static_cast<uint32_t>(
                __builtin_bit_cast(uint16_t, static_cast<_Float16>(-1024.0f * static_cast<float>(sc))));
            const uint32_t nb2 = nbh | (nbh << 16);
            const uint32_t mnh = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(static_cast<float>(mn))));
            const uint32_t mn2 = mnh | (mnh << 16);
            const half8 bm = __builtin_bit_cast(half8, u32x4v{mn2, mn2, mn2, mn2});
            const uint32_t w[4] = {qw[cc].x, qw[cc].y, qw[cc].z, qw[cc].w};
            half8 bq[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const uint32_t w0 = (w[2 * jj] >> nsh) & 0x0f0f0f0fu, w1 = (w[2 * jj + 1] >> nsh) & 0x0f0f0f0fu;
                bq[jj] = __builtin_bit_cast(half8, u32x4v{gg_hfma(gg_magic<0>(w0), sc2, nb2), gg_hfma(gg_magic<1>(w0), sc2, nb2),
                                                          gg_hfma(gg_magic<0>(w1), sc2, nb2), gg_hfma(gg_magic<1>(w1), sc2, nb2)});
            }
            const bool has_min = (mn0 | mn1) != 0;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const half8 x0 = __builtin_bit_cast(half8, raw[mt][cc][0]), x1 = __builtin_bit_cast(half8, raw[mt][cc][1]);
                f32x4m cq = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, bq[0], z4, 0, 0, 0);
                cq = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, bq[1], cq, 0, 0, 0);
                f32x4m cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, bm, z4, 0, 0, 0);
                cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, bm, cm, 0, 0, 0);
                const float dm = has_min ? dmin : 0.0f;
                acc[mt].x = fmaf(dd, cq.x, acc[mt].x) - (has_min ? dm * cm.x : 0.0f);
                acc[mt].y = fmaf(dd, cq.y, acc[mt].y) - (has_min ? dm * cm.y : 0.0f);
                acc[mt].z = fmaf(dd, cq.z, acc[mt].z) - (has_min ? dm * cm.z : 0.0f);
                acc[mt].w = fmaf(dd, cq.w, acc[mt].w) - (has_min ? dm * cm.w : 0.0f);
            }
        }

        if constexpr (RT > 0) {
#pragma unroll
            for (int t = 0; t < RT; ++t)
                if (t == nt)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) keep[t][mt] = acc[mt];
            ++nt;
        } else {
            const uint32_t rb = GL::kRedOff + buf * GL::kRedBuf;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) *lds<lds_f32x4m>(rb + ((wave * MT + mt) * 64 + lane) * 16) = acc[mt];
            lds_barrier();
            gemm_tile_out<MT>(a, rb, tile, tid);
        }
        buf ^= 1;
        slot = slot + 1 == D ? 0 : slot + 1;
        tile += stride;
        if (--left < 0) break;
    }
    wait_vmcnt<0>();                             // no LDS-DMA write may land after the wave ends (or in the reduction)
    if constexpr (RT > 0) {
        lds_barrier();
#pragma unroll
        for (int t = 0; t < RT; ++t)
            if (t < nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    *lds<lds_f32x4m>(t * (kGemmWaves * MT * 1024) + ((wave * MT + mt) * 64 + lane) * 16) = keep[t][mt];
        lds_barrier();
        for (int t = 0; t < nt; ++t)
            gemm_tile_out<MT>(a, t * (kGemmWaves * MT * 1024), blockIdx.y + t * stride, tid);
    }
}

}  // namespace

// The activation-stationary NF4 GEMM's plan for N stacked rows over K with
// passes of M <= 64 tokens on `cus` CUs: MT 16-token tiles, NB 64-element
// blocks per wave (K % (512 * NB) == 0; MT * NB <= 8 keeps the fragments in
// registers), `slices` = K / (512 * NB) workgroup K slices and `groups`
// workgroups per slice, each walking every groups-th 16-row tile. False when
// the shape does not fit the kernel.
bool nf4_gemm_plan(int N, int K, int M, int cus, int &mt, int &nb, int &slices, int &groups) {
    if (M < 1 || M > 64 || K % 1024 != 0 || N < 1) return false;
    mt = (M + 15) / 16;
    const int nbmax = 8 / mt;
    const int kc = K / 512;
    static const int cand[] = {8, 4, 2};
    nb = 0;
    for (int c : cand)
        if (c <= nbmax && kc % c == 0) {
            nb = c;
            break;
        }
    if (nb == 0) return false;
    slices = kc / nb;
    const int tiles = (N + 15) / 16;
    int gr = cus / slices;
    if (gr < 1) gr = 1;
    if (gr > tiles) gr = tiles;
    const int per = (tiles + gr - 1) / gr;
    groups = (tiles + per - 1) / per;
    return groups <= 65535;
}

size_t nf4_xpack_bytes(int M, int K) { return static_cast<size_t>((M + 15) / 16) * K * 32; }

int nf4_gemm_pass(const RowsOut *outs, int nseg, const float *A, int K, int M, bool add, float *part,
                  size_t part_floats, const SliceTail *tail, const uint16_t *xpacked) {
    GemmArgs args{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const RowsOut &o = outs[i];
            if (i < nseg - 1 && o.n % 16 != 0) return ALJABR_ROCM_ERR_UNSUPPORTED;
            end += o.n;
            if (end > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.y[i] = o.y;
            args.w[i] = o.w;
            args.absmax[i] = o.absmax;
            args.end[i] = static_cast<int>(end);
        } else {
            args.end[i] = 0x7fffffff;
        }
    }
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    int mt = 0, nb = 0, slices = 0, groups = 0;
    if (!nf4_gemm_plan(static_cast<int>(end), K, M, cus, mt, nb, slices, groups)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    args.tiles = (args.N + 15) / 16;
    args.add = slices == 1 && add;
    // One buffer: the slice partials (when K is split or a tail follows),
    // then the activations' fp16 fragment image (mt * K * 32 bytes, 256-byte
    // aligned): the caller's `part` when it holds both, else the stream's.
    const size_t pfl = slices > 1 || tail ? static_cast<size_t>(slices) * M * args.N : 0;
    const size_t xoff = (pfl + 63) & ~static_cast<size_t>(63);
    const size_t need = xpacked ? pfl : xoff + static_cast<size_t>(mt) * K * 8;
    float *buf = !need ? nullptr
                 : part && need <= part_floats ? part
                                               : static_cast<float *>(stream_scratch(need * sizeof(float), kScratchPartials));
    if (need && !buf) return ALJABR_ROCM_ERR_BUFFER;
    args.part = pfl ? buf : nullptr;
    args.xp = xpacked ? reinterpret_cast<const u32x4v *>(xpacked) : reinterpret_cast<const u32x4v *>(buf + xoff);
    const dim3 grid(static_cast<unsigned>(slices), static_cast<unsigned>(groups));
    hipStream_t s = current_stream();
    if (!xpacked) {
        const int total = mt * (K / 64) * 128;
        hipLaunchKernelGGL(nf4_xpack_kernel, dim3((total + 255) / 256), dim3(256), 0, s, A,
                           reinterpret_cast<u32x4v *>(buf + xoff), M, K, total);
    }
    // Partial tiles kept in registers to the end when a workgroup walks at
    // most RT tiles and the RT x MT accumulators fit beside the fragments
    // (RT = 4, or 8 for MT = 1 with NB <= 4; MT = 2 only with NB = 2), else
    // summed after every tile.
    const int per = (args.tiles + groups - 1) / groups;
    const int rt = mt == 1 ? (per <= 4 ? 4 : per <= 8 && nb <= 4 ? 8 : 0) : mt == 2 && nb == 2 && per <= 4 ? 4 : 0;
    const void *fn = nullptr;
    uint32_t lds_bytes = 0;
#define ALJ_GEMM_CASE(MT_, NB_, RT_)                                                     \
    if (mt == MT_ && nb == NB_ && rt == RT_) {                                           \
        fn = reinterpret_cast<const void *>(nf4_gemm_kernel<MT_, NB_, RT_>);             \
        lds_bytes = GemmLds<MT_, NB_>::kBytes;                                           \
    }
    ALJ_GEMM_CASE(1, 2, 0) ALJ_GEMM_CASE(1, 4, 0) ALJ_GEMM_CASE(1, 8, 0)
    ALJ_GEMM_CASE(1, 2, 4) ALJ_GEMM_CASE(1, 4, 4) ALJ_GEMM_CASE(1, 8, 4)
    ALJ_GEMM_CASE(1, 2, 8) ALJ_GEMM_CASE(1, 4, 8)
    ALJ_GEMM_CASE(2, 2, 0) ALJ_GEMM_CASE(2, 4, 0)
    ALJ_GEMM_CASE(2, 2, 4)
    ALJ_GEMM_CASE(3, 2, 0)
    ALJ_GEMM_CASE(4, 2, 0)
#undef ALJ_GEMM_CASE
    if (!fn) return ALJABR_ROCM_ERR_UNSUPPORTED;
    static std::atomic<bool> lds_set[5][9][9];   // per (MT, NB, RT): the attribute is per kernel, per process
    if (!lds_set[mt][nb][rt].load(std::memory_order_acquire)) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
        lds_set[mt][nb][rt].store(true, std::memory_order_release);
    }
    void *kargs[] = {&args};
    hipError_t e = hipLaunchKernel(fn, grid, dim3(kGemmThreads), kargs, lds_bytes, s);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "nf4 gemm launch: %s", hipGetErrorString(e));
    if (tail) return enqueue_slice_tail(*tail, args.part, slices, M, args.N);
    if (slices > 1) return enqueue_slice_sum(args.y, args.end, nseg, M, args.N, args.part, slices, add);
    return ALJABR_ROCM_OK;
}

// GGUF Q4_0 / Q8_0 pass of M <= 16 tokens on gguf_gemm_kernel: K slices of
// 8 waves x 512 elements (Q4_0, K % 4096 == 0) or x 256 (K % 2048 == 0), the
// workgroups of a slice walking every groups-th 16-row tile; one slice
// writes (or adds into) the outputs, several store partials for the slice
// sum or the tail. UNSUPPORTED when the shape does not fit.
int gguf_gemm_pass(const RowsOut *outs, int nseg, const float *A, int K, int type, int M, bool add, float *part,
                   size_t part_floats, const SliceTail *tail) {
    if ((type != ALJABR_ROCM_TYPE_Q4_0 && type != ALJABR_ROCM_TYPE_Q8_0) || M < 1 || M > 16 || nseg < 1 ||
        nseg > 3 || !aligned(A, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    // Q8_0's 34-byte blocks leave no registers for 16 blocks a wave.
    const int nbk = K % 4096 == 0 && type == ALJABR_ROCM_TYPE_Q4_0 ? 16 : K % 2048 == 0 ? 8 : 0;
    if (nbk == 0) return ALJABR_ROCM_ERR_UNSUPPORTED;
    GemmArgs args{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const RowsOut &o = outs[i];
            if (o.n <= 0 || (i < nseg - 1 && o.n % 16 != 0)) return ALJABR_ROCM_ERR_UNSUPPORTED;
            end += o.n;
            if (end > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.y[i] = o.y;
            args.w[i] = o.w;
            args.end[i] = static_cast<int>(end);
        } else {
            args.end[i] = 0x7fffffff;
        }
    }
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int slices = K / (8 * 32 * nbk);
    const int tiles = static_cast<int>((end + 15) / 16);
    int gr = cus / slices;
    if (gr < 1) gr = 1;
    if (gr > tiles) gr = tiles;
    const int per = (tiles + gr - 1) / gr;
    const int groups = (tiles + per - 1) / per;
    // A walk of one or two tiles pays the activation loads and the wave
    // reduction for too few weight bytes: the LDS-staged kernel does better.
    if (per < 3 || groups > 65535) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    args.tiles = tiles;
    args.add = slices == 1 && add && !tail;
    const size_t pfl = slices > 1 || tail ? static_cast<size_t>(slices) * M * args.N : 0;
    float *buf = !pfl ? nullptr
                 : part && pfl <= part_floats ? part
                                              : static_cast<float *>(stream_scratch(pfl * sizeof(float), kScratchPartials));
    if (pfl && !buf) return ALJABR_ROCM_ERR_BUFFER;
    args.part = buf;
    const int rt = per <= 4 ? 4 : per <= 8 && nbk == 8 ? 8 : 0;
    const int f = type == ALJABR_ROCM_TYPE_Q4_0 ? 0 : 1;
    const void *fn = nullptr;
    uint32_t lds_bytes = 0;
#define ALJ_GG_CASE(F_, NBK_, RT_)                                                       \
    if (f == F_ && nbk == NBK_ && rt == RT_) {                                           \
        fn = reinterpret_cast<const void *>(gguf_gemm_kernel<F_, NBK_, RT_>);            \
        lds_bytes = GgLds<F_, NBK_>::kBytes;                                             \
    }
    ALJ_GG_CASE(0, 16, 0) ALJ_GG_CASE(0, 16, 4) ALJ_GG_CASE(0, 8, 0) ALJ_GG_CASE(0, 8, 4) ALJ_GG_CASE(0, 8, 8)
    ALJ_GG_CASE(1, 8, 0) ALJ_GG_CASE(1, 8, 4) ALJ_GG_CASE(1, 8, 8)
#undef ALJ_GG_CASE
    if (!fn) return ALJABR_ROCM_ERR_UNSUPPORTED;
    static std::atomic<bool> lds_set[2][17][9];  // per (format, NBK, RT): the attribute is per kernel, per process
    if (!lds_set[f][nbk][rt].load(std::memory_order_acquire)) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
        lds_set[f][nbk][rt].store(true, std::memory_order_release);
    }
    void *kargs[] = {&args};
    const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(slices), static_cast<unsigned>(groups)),
                                         dim3(kGemmThreads), kargs, lds_bytes, current_stream());
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "gguf gemm launch: %s", hipGetErrorString(e));
    if (tail) return enqueue_slice_tail(*tail, args.part, slices, M, args.N);
    if (slices > 1) return enqueue_slice_sum(args.y, args.end, nseg, M, args.N, args.part, slices, add);
    return ALJABR_ROCM_OK;
}

// Q4_K pass of M <= 64 tokens on q4k_gemm_kernel: K slices of 8 waves x NSB
// 256-element super-blocks (NSB 2 for up to 32 tokens, else 1; K % 4096 ==
// 0: with one super-block per wave the extra slices and their sum cost more
// than the LDS-staged kernel's time on the Llama shapes), the workgroups of a
// slice walking
// every groups-th 16-row tile; the fp16 A image built first (or passed in
// `xpacked`), one buffer holding the slice partials (several slices or a
// tail) and the image, as nf4_gemm_pass. UNSUPPORTED when the shape does not
// fit or a workgroup's walk is shorter than three tiles.
int q4k_gemm_pass(const RowsOut *outs, int nseg, const float *A, int K, int M, bool add, float *part,
                  size_t part_floats, const SliceTail *tail, const uint16_t *xpacked) {
    if (M < 1 || M > 64 || nseg < 1 || nseg > 3 || K % 4096 != 0 || !aligned(A, 16)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    GemmArgs args{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const RowsOut &o = outs[i];
            if (o.n <= 0 || (i < nseg - 1 && o.n % 16 != 0)) return ALJABR_ROCM_ERR_UNSUPPORTED;
            end += o.n;
            if (end > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.y[i] = o.y;
            args.w[i] = o.w;
            args.end[i] = static_cast<int>(end);
        } else {
            args.end[i] = 0x7fffffff;
        }
    }
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const int mt = (M + 15) / 16;
    const int nsb = mt <= 2 ? 2 : 1;
    const int slices = K / (2048 * nsb);
    const int tiles = static_cast<int>((end + 15) / 16);
    int gr = cus / slices;
    if (gr < 1) gr = 1;
    if (gr > tiles) gr = tiles;
    const int per = (tiles + gr - 1) / gr;
    const int groups = (tiles + per - 1) / per;
    if (per < 3 || groups > 65535) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    args.tiles = tiles;
    args.add = slices == 1 && add && !tail;
    const size_t pfl = slices > 1 || tail ? static_cast<size_t>(slices) * M * args.N : 0;
    const size_t xoff = (pfl + 63) & ~static_cast<size_t>(63);
    const size_t need = xpacked ? pfl : xoff + static_cast<size_t>(mt) * K * 8;
    float *buf = !need ? nullptr
                 : part && need <= part_floats ? part
                                               : static_cast<float *>(stream_scratch(need * sizeof(float), kScratchPartials));
    if (need && !buf) return ALJABR_ROCM_ERR_BUFFER;
    args.part = pfl ? buf : nullptr;
    args.xp = xpacked ? reinterpret_cast<const u32x4v *>(xpacked) : reinterpret_cast<const u32x4v *>(buf + xoff);
    hipStream_t s = current_stream();
    const int rt = mt == 1 ? (per <= 4 ? 4 : per <= 8 ? 8 : 0) : mt == 2 && nsb == 1 && per <= 4 ? 4 : 0;
    const void *fn = nullptr;
    uint32_t lds_bytes = 0;
#define ALJ_Q4K_CASE(MT_, NSB_, RT_)                                                      \
    if (mt == MT_ && nsb == NSB_ && rt == RT_) {                                           \
        fn = reinterpret_cast<const void *>(q4k_gemm_kernel<MT_, NSB_, RT_>);              \
        lds_bytes = Q4kLds<MT_, NSB_>::kBytes;                                             \
    }
    ALJ_Q4K_CASE(1, 2, 0) ALJ_Q4K_CASE(1, 2, 4) ALJ_Q4K_CASE(1, 2, 8) ALJ_Q4K_CASE(2, 2, 0)
    ALJ_Q4K_CASE(3, 1, 0) ALJ_Q4K_CASE(4, 1, 0)
#undef ALJ_Q4K_CASE
    if (!fn) return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (!xpacked) {
        const int total = mt * (K / 64) * 128;
        hipLaunchKernelGGL(nf4_xpack_kernel, dim3((total + 255) / 256), dim3(256), 0, s, A,
                           reinterpret_cast<u32x4v *>(buf + xoff), M, K, total);
    }
    static std::atomic<bool> lds_set[5][3][9];   // per (MT, NSB, RT): the attribute is per kernel, per process
    if (!lds_set[mt][nsb][rt].load(std::memory_order_acquire)) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
        lds_set[mt][nsb][rt].store(true, std::memory_order_release);
    }
    void *kargs[] = {&args};
    const hipError_t e = hipLaunchKernel(fn, dim3(static_cast<unsigned>(slices), static_cast<unsigned>(groups)),
                                         dim3(kGemmThreads), kargs, lds_bytes, s);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "q4_k gemm launch: %s", hipGetErrorString(e));
    if (tail) return enqueue_slice_tail(*tail, args.part, slices, M, args.N);
    if (slices > 1) return enqueue_slice_sum(args.y, args.end, nseg, M, args.N, args.part, slices, add);
    return ALJABR_ROCM_OK;
}

size_t q4k_gemm_scratch_floats(int M, int N, int K) {
    if (M < 1 || K % 4096 != 0) return 0;
    const int m = M > 64 ? 64 : M;
    const size_t pfl = static_cast<size_t>(K / (m <= 32 ? 4096 : 2048)) * m * N;
    return ((pfl + 63) & ~static_cast<size_t>(63)) + static_cast<size_t>((m + 15) / 16) * K * 8;
}

// The largest buffer a pass of enqueue_nf4_mfma_multi takes: for the
// register-resident kernel the slice partials (counted as when a tail
// follows) and the fp16 activation image after them, for the LDS-staged one
// the slice partials.
size_t nf4_mfma_scratch_floats(int M, int N, int K) {
    if (M < 2 || N < 1 || K % kSub != 0) return 0;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    size_t need = 0;
    for (int m0 = 0; m0 < M; m0 += 64) {
        const int mm = M - m0 < 64 ? M - m0 : 64;
        int mt = 0, nb = 0, slices = 0, groups = 0;
        size_t p;
        if (nf4_gemm_plan(N, K, mm, cus, mt, nb, slices, groups)) {
            const size_t pfl = static_cast<size_t>(slices) * mm * N;
            p = ((pfl + 63) & ~static_cast<size_t>(63)) + static_cast<size_t>(mt) * K * 8;
        } else {
            int nt = 1, q = 1;
            nf4_mfma_plan(N, K, mm, cus, nt, q);
            const int nsub = K / kSub;
            if (q > nsub) q = nsub;
            p = static_cast<size_t>((nsub + q - 1) / q) * mm * N;
        }
        if (p > need) need = p;
    }
    return need;
}

// Row tiles per wave and sub-slices per slice for N stacked rows over K on
// `cus` CUs, for passes of M tokens: two tiles per wave (each activation
// fragment read from LDS feeds two tiles) once the 512-row groups number
// at least 16 and a pass has one token tile (M <= 32; two token tiles take
// the registers a second row tile would), and the fewest slices that still
// give every CU a workgroup (one workgroup fits a CU).
void nf4_mfma_plan(int N, int K, int M, int cus, int &nt, int &q) {
    const int nsub = K / kSub;
    nt = M <= 32 && (N + 2LL * kGroupRows - 1) / (2LL * kGroupRows) >= 16 ? 2 : 1;
    const long long groups = (N + static_cast<long long>(kGroupRows) * nt - 1) / (static_cast<long long>(kGroupRows) * nt);
    q = nsub;
    for (int cand = 1; cand < nsub; ++cand) {
        if (groups * ((nsub + cand - 1) / cand) <= cus) {
            q = cand;
            break;
        }
    }
}

// The GEMM pass of M <= 64 tokens with an explicit plan (nt = 1 or 2 row
// tiles per wave, q >= 1 sub-slices per slice; nt = 1 when M > 32: two
// token tiles).
int nf4_mfma_pass_planned(const RowsOut *outs, int nseg, const float *A, int K, int M, bool add, float *part,
                          size_t part_floats, int nt, int q, const SliceTail *tail) {
    MmArgs args{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const RowsOut &o = outs[i];
            end += o.n;
            if (end > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
            args.y[i] = o.y;
            args.w[i] = o.w;
            args.absmax[i] = o.absmax;
            args.end[i] = static_cast<int>(end);
        } else {
            args.end[i] = 0x7fffffff;
        }
    }
    if ((nt != 1 && nt != 2) || q < 1 || M < 1 || M > 64 || (M > 32 && nt != 1)) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    const int nsub = K / kSub;
    if (q > nsub) q = nsub;
    args.q = q;
    const int slices = (nsub + q - 1) / q;
    const long long groups = (args.N + static_cast<long long>(kGroupRows) * nt - 1) / (static_cast<long long>(kGroupRows) * nt);
    if (groups > 65535) return ALJABR_ROCM_ERR_UNSUPPORTED;
    args.add = slices == 1 && add;
    if (slices > 1 || tail) {
        const size_t need = static_cast<size_t>(slices) * M * args.N;
        args.part = part && need <= part_floats
                        ? part
                        : static_cast<float *>(stream_scratch(need * sizeof(float), kScratchPartials));
        if (!args.part) return ALJABR_ROCM_ERR_BUFFER;
    }
    hipStream_t s = current_stream();
    static bool lds_set = false;                 // the attribute is per kernel, per process
    if (!lds_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(nf4_mm_kernel<1, 1>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(Lds<1>::kBytes));
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(nf4_mm_kernel<2, 1>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(Lds<1>::kBytes));
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(nf4_mm_kernel<1, 2>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(Lds<2>::kBytes));
        lds_set = true;
    }
    const dim3 grid(slices, static_cast<unsigned>(groups));
    if (M > 32) hipLaunchKernelGGL((nf4_mm_kernel<1, 2>), grid, dim3(kMmThreads), Lds<2>::kBytes, s, args);
    else if (nt == 2) hipLaunchKernelGGL((nf4_mm_kernel<2, 1>), grid, dim3(kMmThreads), Lds<1>::kBytes, s, args);
    else hipLaunchKernelGGL((nf4_mm_kernel<1, 1>), grid, dim3(kMmThreads), Lds<1>::kBytes, s, args);
    if (tail) return enqueue_slice_tail(*tail, args.part, slices, M, args.N);
    if (slices > 1) return enqueue_slice_sum(args.y, args.end, nseg, M, args.N, args.part, slices, add);
    return ALJABR_ROCM_OK;
}

int enqueue_slice_sum(float *const *ys, const int *ends, int nseg, int M, int N, const float *part, int slices,
                      bool add) {
    ReduceArgs red{};
    for (int i = 0; i < 3; ++i) {
        red.y[i] = i < nseg ? ys[i] : nullptr;
        red.end[i] = i < nseg ? ends[i] : 0x7fffffff;
    }
    red.nseg = nseg;
    red.M = M;
    red.N = N;
    red.slices = slices;
    red.add = add ? 1 : 0;
    red.part = part;
    const long long total = static_cast<long long>(M) * N;
    hipLaunchKernelGGL(nf4_mm_reduce_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       current_stream(), red);
    return ALJABR_ROCM_OK;
}

int enqueue_nf4_mfma_multi(const RowsOut *outs, int nseg, const float *A, int K, int bs_shift, int M, bool add,
                           float *part, size_t part_floats, const SliceTail *tail, const uint16_t *xpacked) {
    if (nseg < 1 || nseg > 3 || M < 2 || K % kSub != 0 || bs_shift != 6 || !aligned(A, 16) || (tail && M > 64))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    long long n = 0;
    for (int i = 0; i < nseg; ++i) {
        if (outs[i].n <= 0 || !aligned(outs[i].w, 16) || !aligned(outs[i].absmax, 8) ||
            (i < nseg - 1 && outs[i].n % 32 != 0))
            return ALJABR_ROCM_ERR_UNSUPPORTED;
        n += outs[i].n;
    }
    if (n > 0x7fff0000LL) return ALJABR_ROCM_ERR_UNSUPPORTED;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    // Passes of up to 64 tokens (two token tiles); a pass's outputs are the
    // rows m0 .. m0 + mm - 1 of each segment.
    for (int m0 = 0; m0 < M; m0 += 64) {
        const int mm = M - m0 < 64 ? M - m0 : 64;
        int nt = 1, q = 1;
        nf4_mfma_plan(static_cast<int>(n), K, mm, cus, nt, q);
        RowsOut o[3];
        for (int i = 0; i < nseg; ++i) {
            o[i] = outs[i];
            o[i].y = outs[i].y + static_cast<size_t>(m0) * outs[i].n;
        }
        // The register-resident kernel where the shape fits it, else the
        // LDS-staged one (K % 256 == 0, fp32-accurate).
        {
            const int rc = nf4_gemm_pass(o, nseg, A + static_cast<size_t>(m0) * K, K, mm, add, part, part_floats, tail,
                                         M <= 64 ? xpacked : nullptr);
            if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) {
                if (rc != ALJABR_ROCM_OK) return rc;
                continue;
            }
        }
        const int rc = nf4_mfma_pass_planned(o, nseg, A + static_cast<size_t>(m0) * K, K, mm, add, part, part_floats,
                                             nt, q, tail);
        if (rc != ALJABR_ROCM_OK) return rc;
    }
    return ALJABR_ROCM_OK;
}

int enqueue_nf4_mfma(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M, bool add, float *part, size_t part_floats) {
    const RowsOut o{C, Bq, absmax, N};
    return enqueue_nf4_mfma_multi(&o, 1, A, K, bs_shift, M, add, part, part_floats);
}

}  // namespace aljabr
