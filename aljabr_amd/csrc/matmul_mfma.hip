// matmul_mfma.hip - NF4 small-M GEMM on the matrix cores:
// Y[M,N] = X[M,K] . W[N,K]^T for 2 <= M <= 64 (a prompt chunk or a decode
// batch), W in NF4 (STC/DequantizationKernel.java:84-102). Replaces the
// reference's per-token loop over the matvec (MTLJ/MetalComputeBackend.java:
// 435-470): W is read from HBM once for all M tokens.
//
// MFMA v_mfma_f32_32x32x16_f16 with A = X (32 token rows per m-tile) and
// B = W^T (32 weight rows per wave as the 32 output columns), fp32
// accumulation. Both operands are fp16: NF4 levels rounded to fp16 (relative
// error <= 2^-11) and activations rounded to fp16; the per-block absmax stays
// fp32 and is applied to the fp32 accumulators once per 64-element block
// (C += s * C_block), so no product is rounded through fp16 twice.
//
// Decode: a code byte (two weights) indexes a 256-entry table of packed fp16
// level pairs in LDS, which is exactly one B-operand register. The table is
// replicated 64 times, entry e of replica r at byte e*256 + r*4, so lane l
// reads replica l and a wave never conflicts; the address is one v_perm_b32.
//
// Operand layout (32x32x16): lane l supplies A[m = l%32][8*(l/32) + e] and
// B[8*(l/32) + e][n = l%32], e = 0..7; accumulator r of lane l is
// C[8*(r/4) + 4*(l/32) + r%4][l%32]. The contraction index k' is mapped to
// the real K so that one MFMA step covers 16 elements of one 64-element
// block, and each lane reads 16 contiguous code bytes per block: for block
// b of a 256-element iteration and step j (0..3) of the block, lane half h
// supplies k = 64b + 32h + 8j + e.
//
// Work split: a workgroup is 8 waves x 32 rows = 256 rows of W and one
// K-slice of KS elements; slices add their partial sums into Y with
// hardware float atomics (Y is zeroed first), so results are exact up to
// fp32 summation order, which varies between runs.
#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr int kMmWaves = 8;
constexpr int kMmThreads = kMmWaves * 64;
constexpr int kMmRowsPerWg = kMmWaves * 32;
constexpr int kTableBytes = 256 * 64 * 4;       // 256 entries x 64 replicas x fp16 pair

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
    int M, N, K, bs_shift;   // N: stacked rows
};

// The segment of a tile starting at stacked row r0 (past the end: the last
// segment, with local rows past its end).
struct TileRef {
    const uint8_t *w;
    const float *absmax;
    float *y;
    int local0, n;
};

__device__ __forceinline__ TileRef tile_ref(const MmArgs &a, int r0) {
    int s = (r0 >= a.end[0]) + (r0 >= a.end[1]);
    if (s > a.nseg - 1) s = a.nseg - 1;
    const int start = s == 0 ? 0 : s == 1 ? a.end[0] : a.end[1];
    TileRef t;
    t.w = s == 0 ? a.w[0] : s == 1 ? a.w[1] : a.w[2];
    t.absmax = s == 0 ? a.absmax[0] : s == 1 ? a.absmax[1] : a.absmax[2];
    t.y = s == 0 ? a.y[0] : s == 1 ? a.y[1] : a.y[2];
    t.local0 = r0 - start;
    t.n = (s == 0 ? a.end[0] : s == 1 ? a.end[1] : a.end[2]) - start;
    return t;
}

__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
    const _Float16 a = static_cast<_Float16>(lo), b = static_cast<_Float16>(hi);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
}

// B fragment (8 fp16 weights) for code dword `w`: byte t holds elements
// 2t (high nibble) and 2t+1 (low nibble). Table entry e of replica r is at
// byte e*256 + r*4: v_perm puts the code byte in bits 8-15 and r*4 (cl) in
// bits 0-7.
__device__ __forceinline__ uint32_t pair16_at(const char *tbl, uint32_t addr) {
    return *reinterpret_cast<const uint32_t *>(tbl + addr);
}
__device__ __forceinline__ half8 decode8(uint32_t w, uint32_t cl, const char *tbl) {
    u32x4v r;
    r.x = pair16_at(tbl, __builtin_amdgcn_perm(w, cl, 0x0C0C0400u));
    r.y = pair16_at(tbl, __builtin_amdgcn_perm(w, cl, 0x0C0C0500u));
    r.z = pair16_at(tbl, __builtin_amdgcn_perm(w, cl, 0x0C0C0600u));
    r.w = pair16_at(tbl, __builtin_amdgcn_perm(w, cl, 0x0C0C0700u));
    return __builtin_bit_cast(half8, r);
}

// Pair table: dword slot i = e*64 + r. Thread tid (of 512) fills slots
// tid + 512k (k < 32): e = tid/64 + 8k, so its low nibble is tid/64 + 8*(k
// odd) and its high nibble k/2.
__device__ __forceinline__ void build_pair16_table(uint32_t *tbl_s, int tid) {
    const float lo_a = nf4_level_sel(tid >> 6), lo_b = nf4_level_sel((tid >> 6) + 8);
    constexpr float kNF4[16] = {
        -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
#pragma unroll
    for (int k = 0; k < 32; ++k) tbl_s[tid + kMmThreads * k] = pack_half2(kNF4[k >> 1], (k & 1) ? lo_b : lo_a);
}

// Loads of one work unit, coalesced (8 lanes read a whole 128-byte row
// segment; the MFMA layout would touch 32 lines per instruction and stall
// the texture path): instruction i covers rows 8i + lane/8 of the wave's
// 32-row tile, bytes 16*(lane%8) of iteration it's segment. The first unit
// of a tile also loads its SB scales: lane covers row lane/2, half lane%2.
template <int ITERS, int SB>
__device__ __forceinline__ void issue_unit(u32x4 (&q)[4], float (&sc)[SB / 2], const MmArgs &a, const TileRef &tr,
                                           int it, int ks0, int lane) {
    if (it == 0) {
        const int srow = min(tr.local0 + (lane >> 1), tr.n - 1);
        const float *sp = tr.absmax + ((static_cast<size_t>(srow) * a.K + ks0) >> 6) + (SB / 2) * (lane & 1);
        if constexpr (SB / 2 == 4) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(sp);
            sc[0] = v.x; sc[1] = v.y; sc[2] = v.z; sc[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < SB / 2; ++j) sc[j] = sp[j];
        }
    }
    const size_t row_bytes = static_cast<size_t>(a.K) >> 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = min(tr.local0 + 8 * i + (lane >> 3), tr.n - 1);
        q[i] = *reinterpret_cast<const u32x4 *>(tr.w + row * row_bytes + (ks0 >> 1) + 128 * it + 16 * (lane & 7));
    }
    __builtin_amdgcn_sched_barrier(0);           // keep units in issue order
}

template <int MT, int KS>
constexpr size_t mm_lds_bytes() {
    // x slice (fp16, padded rows) + per-wave code staging (32 rows x 144 B)
    // + per-wave scale staging (32 rows x KS/64 floats).
    return static_cast<size_t>(32 * MT) * (KS + 8) * 2 + kMmWaves * 32 * 144 + kMmWaves * 32 * (KS / 64) * 4;
}

template <int MT, int KS, int NT>
__global__ __launch_bounds__(kMmThreads) void nf4_mm_kernel(MmArgs a) {
    constexpr int ITERS = KS / 256;
    constexpr int SB = KS / 64;                  // 64-element blocks (absmax scales) per row and slice
    constexpr int RS = KS + 8;                   // x row stride in halves (16-byte pad: conflict-free reads)
    extern __shared__ uint8_t smem[];
    __shared__ uint32_t tbl_s[kTableBytes / 4];  // static: its LDS address is a known constant
    const char *tbl = reinterpret_cast<const char *>(tbl_s);
    _Float16 *xs = reinterpret_cast<_Float16 *>(smem);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;
    const int nl = lane & 31;                    // this lane's output column (weight row) in a tile
    uint8_t *cstage = smem + static_cast<size_t>(32 * MT) * RS * 2 + wave * (32 * 144);
    float *sstage = reinterpret_cast<float *>(smem + static_cast<size_t>(32 * MT) * RS * 2 + kMmWaves * 32 * 144) +
                    wave * (32 * SB);
    const int ks0 = blockIdx.y * KS;

    // Activation slice.
    constexpr int XF4 = 32 * MT * (KS / 4) / kMmThreads;
    static_assert(32 * MT * (KS / 4) % kMmThreads == 0, "x slice split");
    f32x4 xv[XF4];
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
        const int i = tid + kMmThreads * j;
        const int m = min(i / (KS / 4), a.M - 1), c = i % (KS / 4);
        xv[j] = *reinterpret_cast<const f32x4 *>(a.x + static_cast<size_t>(m) * a.K + ks0 + 4 * c);
    }

    // x slice -> fp16 rows [32*MT][KS] (rows >= M are zero). Staged before
    // the weight loads go out: behind 30 MB of weight requests the activation
    // loads would wait several microseconds.
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
        const int i = tid + kMmThreads * j;
        const int m = i / (KS / 4), c = i % (KS / 4);
        f32x4 v = xv[j];
        if (m >= a.M) v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        *reinterpret_cast<uint2 *>(xs + m * RS + 4 * c) = make_uint2(pack_half2(v.x, v.y), pack_half2(v.z, v.w));
    }
    __builtin_amdgcn_sched_barrier(0);           // the weight loads must not move above this

    // Weights, all issued up front and coalesced (whole 128-byte row segments per
    // 8 lanes; the MFMA layout would touch 32 lines per instruction and stall
    // the texture path): codes of iteration it, instruction i: row
    // 8i + lane/8 of the wave's tile, bytes 16*(lane%8) of the segment; the
    // row's SB scales: lane covers row lane/2, half lane%2.
    // Work units u = (tile t = u / ITERS, iteration it = u % ITERS); loads run
    // W units ahead of the unit being computed, so the memory queue holds a
    // few units per wave instead of the whole slice (issuing everything at
    // once stalls the wave at issue until most of it has arrived).
    constexpr int U = NT * ITERS;
    constexpr int W = 2;
    TileRef tr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) tr[t] = tile_ref(a, blockIdx.x * (kMmRowsPerWg * NT) + t * kMmRowsPerWg + wave * 32);
    u32x4 qc[U][4];
    float sc[NT][SB / 2];
#pragma unroll
    for (int u = 0; u < W && u < U; ++u) issue_unit<ITERS, SB>(qc[u], sc[u / ITERS], a, tr[u / ITERS], u % ITERS, ks0, lane);

    build_pair16_table(tbl_s, tid);
    __syncthreads();

    const uint32_t cl = lane * 4;
    f32x16 acc[MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (u + W < U)
            issue_unit<ITERS, SB>(qc[u + W], sc[(u + W) / ITERS], a, tr[(u + W) / ITERS], (u + W) % ITERS, ks0,
                                      lane);
        const int t = u / ITERS, it = u % ITERS;
        if (it == 0) {
            // Scales of this tile to the MFMA layout: row nl, all SB blocks.
#pragma unroll
            for (int j = 0; j < SB / 2; ++j) sstage[(lane >> 1) * SB + (SB / 2) * (lane & 1) + j] = sc[t][j];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mt][r] = 0.0f;
        }
        // Codes to the MFMA layout through the wave's staging rows (144-byte
        // stride: conflict-free both ways): lane (nl, h) takes bytes
        // 32b + 16h of row nl for block b.
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4 *>(cstage + (8 * i + (lane >> 3)) * 144 + 16 * (lane & 7)) = qc[u][i];
        u32x4 qm[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) qm[b] = *reinterpret_cast<const u32x4 *>(cstage + nl * 144 + 32 * b + 16 * h);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float sblk = sstage[nl * SB + 4 * it + b];
            const uint32_t wd[4] = {qm[b].x, qm[b].y, qm[b].z, qm[b].w};
            f32x16 cb[MT];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half8 bf = decode8(wd[j], cl, tbl);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const _Float16 *xp = xs + (32 * mt + nl) * RS + 256 * it + 64 * b + 32 * h + 8 * j;
                    const half8 af = *reinterpret_cast<const half8 *>(xp);
                    cb[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, j == 0 ? f32x16{} : cb[mt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mt][r] = fmaf(sblk, cb[mt][r], acc[mt][r]);
            // One block at a time: otherwise the scheduler hoists every
            // block's table reads and runs out of registers.
            __builtin_amdgcn_sched_barrier(0);
        }
        if (it == ITERS - 1) {
            const int n = tr[t].local0 + nl;
            if (n < tr[t].n) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int m = 32 * mt + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (m < a.M) unsafeAtomicAdd(tr[t].y + static_cast<size_t>(m) * tr[t].n + n, acc[mt][r]);
                    }
            }
        }
    }
}

__global__ void zero_f32_kernel(float *p, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

template <int MT, int KS, int NT>
void launch_mm(const MmArgs &args, hipStream_t s) {
    static bool lds_set = false;                 // the attribute is per kernel, per process
    const void *fn = reinterpret_cast<const void *>(nf4_mm_kernel<MT, KS, NT>);
    const size_t lds = mm_lds_bytes<MT, KS>();   // + the static table
    if (!lds_set) {
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        lds_set = true;
    }
    const dim3 grid((args.N + kMmRowsPerWg * NT - 1) / (kMmRowsPerWg * NT), args.K / KS), block(kMmThreads);
    hipLaunchKernelGGL((nf4_mm_kernel<MT, KS, NT>), grid, block, lds, s, args);
}

}  // namespace

// M in [2, 64], K % 512 == 0, block size 64, codes, absmax and x 16-byte aligned.
// K-slices of 512 (M <= 32) or 256 (two m-tiles) keep every operand of a
// slice in registers without spills.
int enqueue_nf4_mfma_multi(const RowsOut *outs, int nseg, const float *A, int K, int bs_shift, int M,
                           bool accumulate) {
    if (nseg < 1 || nseg > 3 || M < 2 || M > 64 || K % 512 != 0 || bs_shift != 6 || !aligned(A, 16))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    MmArgs args{};
    long long end = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < nseg) {
            const RowsOut &o = outs[i];
            if (o.n <= 0 || !aligned(o.w, 16) || !aligned(o.absmax, 16) || (i < nseg - 1 && o.n % 32 != 0))
                return ALJABR_ROCM_ERR_UNSUPPORTED;
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
    args.nseg = nseg;
    args.x = A;
    args.M = M;
    args.N = static_cast<int>(end);
    args.K = K;
    args.bs_shift = bs_shift;
    hipStream_t s = current_stream();
    if (!accumulate)   // the K-slices add into the outputs
        for (int i = 0; i < nseg; ++i) {
            const long long total = static_cast<long long>(M) * outs[i].n;
            hipLaunchKernelGGL(zero_f32_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s,
                               outs[i].y, total);
        }
    const int N = args.N;
    const int wgs_n = (N + kMmRowsPerWg - 1) / kMmRowsPerWg;
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    // One generation of workgroups (one per CU): the fewest row tiles per
    // wave (1, 2 or 4) that fit all row tiles x K-slices on the CUs.
    const long long units = static_cast<long long>(wgs_n) * (K / (M <= 32 ? 512 : 256));
    const int nt = units <= cus ? 1 : units <= 2LL * cus ? 2 : 4;
    if (M <= 32) {                               // (four tiles would spill at one m-tile)
        if (nt == 1) launch_mm<1, 512, 1>(args, s);
        else launch_mm<1, 512, 2>(args, s);
    } else {
        if (nt == 1) launch_mm<2, 256, 1>(args, s);
        else if (nt == 2) launch_mm<2, 256, 2>(args, s);
        else launch_mm<2, 256, 4>(args, s);
    }
    return ALJABR_ROCM_OK;
}

int enqueue_nf4_mfma(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M, bool accumulate) {
    const RowsOut o{C, Bq, absmax, N};
    return enqueue_nf4_mfma_multi(&o, 1, A, K, bs_shift, M, accumulate);
}

}  // namespace aljabr
