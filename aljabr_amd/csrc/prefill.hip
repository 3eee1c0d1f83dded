// prefill.hip - prompt (prefill) attention, flash-style on the matrix cores:
// the FA4 entry point of the reference's Metal backend
// (MTLC/aljabr_metal_fa4.m:253-530): out[B,T,H,D] = softmax(scale * Q K^T)
// V per head, Q/out [B,T,H,D], K/V [B,S,H_kv,D], all fp32, H_kv dividing H
// (query head h reads KV head h / (H / H_kv)). Query row t sees keys
// [lo(t), hi(t)): hi = S, or with the causal mask
// min(max(S - T, 0) + t + 1, S) (causal_limit_for_row, aljabr_metal_fa4.m:
// 111-115); lo = 0, or max(hi - window, 0) in the windowed form. A soft cap
// > 0 maps the kept scores to cap * tanh(s / cap) before the softmax.
//
// Fast path (D = 64 or 128): a workgroup is 4 waves x 32 query rows of one
// head and walks the keys in tiles of 32. Each tile of K and V is loaded once
// per workgroup (the next tile's loads in flight during the current tile's
// math), split into fp16 hi + lo parts in LDS (K as [key][d], V transposed
// as [d][key]). A wave computes the transposed score tile S^T = K Q^T with
// v_mfma_f32_32x32x16_f16 (lane l holds 16 keys of query row l % 32, so the
// row's max and sum need one exchange between the two lane halves), keeps
// the online-softmax state per lane, and accumulates O^T = V^T P^T into
// D / 32 accumulator tiles. Every product takes three MFMAs, hi*hi + lo*hi +
// hi*lo, so scores and outputs carry ~2^-22 relative error instead of fp16's
// 2^-11; the key order inside a tile is permuted identically on both sides of
// the P.V contraction to match the score accumulators' layout.
//
// Workgroup order: the KV head varies fastest, so (with H_kv a multiple of 8)
// the workgroups sharing a KV head land on one XCD and its L2; the longest
// (last, under the causal mask) query blocks are dispatched first.
//
// Other head sizes or alignments take fa_generic_kernel (one wave per query
// row, keys in chunks of 1024 through LDS, fp32).
#include <cmath>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2eF = 1.4426950408889634f;
constexpr int kFaWaves = 4;
constexpr int kFaThreads = 64 * kFaWaves;
constexpr int kRowsWg = 32 * kFaWaves;       // query rows per workgroup with one row tile per wave
constexpr int kKeys = 32;                    // keys per tile
constexpr int kVtStride = kKeys + 4;         // halves: 72-byte rows, conflict-free 8-byte reads
constexpr int kGenChunk = 1024;              // generic kernel: keys per LDS chunk

struct FaParams {
    const float *q, *k, *v;
    float *out;
    long long q_b, q_t, q_h;   // element strides of q and out
    long long k_b, k_s, k_h;   // of k and v
    int B, T, S, H, Hkv, G;
    float scale, soft_cap;
    int causal, window;
    int nqb;                   // query blocks (workgroups per batch and head)
};

// Keys [key_lo, key_hi) of query row t; both grow with t.
__device__ __forceinline__ int key_hi(const FaParams &p, int t) {
    if (!p.causal) return p.S;
    const int lim = (p.S > p.T ? p.S - p.T : 0) + t + 1;
    return lim < p.S ? lim : p.S;
}

__device__ __forceinline__ int key_lo(const FaParams &p, int hi) {
    if (p.window <= 0) return 0;
    return hi - p.window > 0 ? hi - p.window : 0;
}

__device__ __forceinline__ void split_half(float v, _Float16 &hi, _Float16 &lo) {
    hi = static_cast<_Float16>(v);
    lo = static_cast<_Float16>(v - static_cast<float>(hi));
}

__device__ __forceinline__ float f4_at(const float4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Scaled score -> log2 domain, with the soft cap on the natural-unit score.
__device__ __forceinline__ float score_log2(float s, float cap) {
    if (cap > 0.0f) s = cap * tanhf(s / cap);
    return s * kLog2eF;
}

// Halves of one tile's LDS image: Kh, Kl as [kKeys][D + 8] and Vh^T, Vl^T
// as [D][kVtStride], padded to whole rounds of 16-byte copies by the
// workgroup (kFaThreads lanes x 8 halves).
template <int D>
constexpr int fa_tile_halves() {
    constexpr int used = 2 * kKeys * (D + 8) + 2 * D * kVtStride;
    constexpr int round = kFaThreads * 8;
    return (used + round - 1) / round * round;
}

// K and V of one (batch, KV head) packed as fp16 hi/lo tiles of kKeys keys
// (keys >= S zero), each the exact byte image of the attention kernel's LDS
// buffer, so that kernel copies tiles into LDS with direct global-to-LDS
// loads. Done once per prefill: the split and the V transpose are not
// repeated by every workgroup that reads a tile.
template <int D>
__global__ __launch_bounds__(256) void fa_pack_kernel(FaParams p, _Float16 *__restrict__ pk, int ntiles) {
    constexpr int KS = D + 8;
    const int tile = blockIdx.x % ntiles;
    const int bk = blockIdx.x / ntiles;                // b * Hkv + kvh
    const int b = bk / p.Hkv, kvh = bk % p.Hkv;
    const float *kbase = p.k + b * p.k_b + kvh * p.k_h;
    const float *vbase = p.v + b * p.k_b + kvh * p.k_h;
    _Float16 *dst = pk + static_cast<long long>(blockIdx.x) * fa_tile_halves<D>();
    const int k0 = tile * kKeys;
    for (int i = threadIdx.x; i < kKeys * (D / 4); i += 256) {
        const int key = i / (D / 4), d4 = i % (D / 4);
        const int kk = k0 + key;
        const float4 a = kk < p.S ? *reinterpret_cast<const float4 *>(kbase + kk * p.k_s + 4 * d4)
                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        half4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            _Float16 x0, x1;
            split_half(f4_at(a, e), x0, x1);
            hi[e] = x0;
            lo[e] = x1;
        }
        *reinterpret_cast<half4 *>(dst + key * KS + 4 * d4) = hi;
        *reinterpret_cast<half4 *>(dst + kKeys * KS + key * KS + 4 * d4) = lo;
    }
    for (int i = threadIdx.x; i < (kKeys / 4) * (D / 4); i += 256) {
        const int kg = i / (D / 4), dg = i % (D / 4);
        float4 r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int kk = k0 + 4 * kg + c;
            r[c] = kk < p.S ? *reinterpret_cast<const float4 *>(vbase + kk * p.k_s + 4 * dg)
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
            half4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 x0, x1;
                split_half(f4_at(r[e], c4), x0, x1);
                hi[e] = x0;
                lo[e] = x1;
            }
            const int d = 4 * dg + c4;
            *reinterpret_cast<half4 *>(dst + 2 * kKeys * KS + d * kVtStride + 4 * kg) = hi;
            *reinterpret_cast<half4 *>(dst + 2 * kKeys * KS + D * kVtStride + d * kVtStride + 4 * kg) = lo;
        }
    }
}

template <int D>
constexpr size_t fa_lds_bytes() {
    return 2 * static_cast<size_t>(fa_tile_halves<D>()) * sizeof(_Float16);   // two tile buffers
}

template <int D, int RT>
__global__ __launch_bounds__(kFaThreads) __attribute__((amdgpu_waves_per_eu(RT == 1 ? 2 : 1, RT == 1 ? 2 : 1))) void fa_prefill_kernel(FaParams p, const _Float16 *__restrict__ pk,
                                                                int ntiles) {
    constexpr int KS = D + 8;                      // K row stride (halves): conflict-free 16-byte reads
    constexpr int STEPS = D / 16;                  // MFMA steps over d for a score tile
    constexpr int DT = D / 32;                     // 32-row d tiles of the output
    constexpr int BUF = fa_tile_halves<D>();      // halves of a packed tile = one LDS buffer
    constexpr int CH = BUF / 8 / kFaThreads;       // 16-byte copies per lane per tile
    constexpr int ROWS_W = 32 * RT, ROWS_WG = ROWS_W * kFaWaves;
    extern __shared__ _Float16 lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, h = lane >> 5, nl = lane & 31;
    int idx = blockIdx.x;
    const int kvh = idx % p.Hkv;
    idx /= p.Hkv;
    const int g = idx % p.G;
    idx /= p.G;
    const int b = idx % p.B;
    idx /= p.B;
    const int qb = p.nqb - 1 - idx;
    const int head = kvh * p.G + g;
    const int t0 = qb * ROWS_WG;
    const int tw = t0 + wave * ROWS_W;
    // This lane's query rows tw + 32u + nl and their key ranges.
    int hi_t[RT], lo_t[RT];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
        const int t = min(tw + 32 * u + nl, p.T - 1);
        hi_t[u] = key_hi(p, t);
        lo_t[u] = key_lo(p, hi_t[u]);
    }
    // Key ranges of the wave (rows tw .. last_w) and of the workgroup, and the
    // band every row of the wave sees whole.
    const bool wave_ok = tw < p.T;
    const int last_w = min(tw + ROWS_W, p.T) - 1;
    const int last_g = min(t0 + ROWS_WG, p.T) - 1;
    const int w_lo = wave_ok ? key_lo(p, key_hi(p, tw)) : 0;
    const int w_hi = wave_ok ? key_hi(p, last_w) : 0;
    const int full_lo = wave_ok ? key_lo(p, key_hi(p, last_w)) : 0;
    const int full_hi = wave_ok ? key_hi(p, tw) : 0;
    const int g_lo = key_lo(p, key_hi(p, t0));
    const int g_hi = key_hi(p, last_g);

    // The lane's query rows times scale * log2(e) as MFMA B fragments: step
    // s holds d = 16s + 8h .. +8, split into hi and lo halves. Scores come
    // out in log2 units; the soft cap is applied in those units too:
    // cap * tanh(s / cap) * log2(e) == c2 * tanh(s2 / c2) with c2 = cap * log2(e).
    half8 qhf[RT][STEPS], qlf[RT][STEPS];
    const float qs = p.scale * kLog2eF;
#pragma unroll
    for (int u = 0; u < RT; ++u) {
        const int t = min(tw + 32 * u + nl, p.T - 1);
        const float *qr = p.q + b * p.q_b + t * p.q_t + head * p.q_h;
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * s + 8 * h);
            const float4 c = *reinterpret_cast<const float4 *>(qr + 16 * s + 8 * h + 4);
            const float vals[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 hi, lo;
                split_half(vals[e] * qs, hi, lo);
                qhf[u][s][e] = hi;
                qlf[u][s][e] = lo;
            }
        }
    }
    const float cap2 = p.soft_cap * kLog2eF;

    const _Float16 *tiles = pk + static_cast<long long>(b * p.Hkv + kvh) * ntiles * BUF;
    // Tile kt into LDS buffer `dst` by direct global-to-LDS copies: copy j of
    // wave w moves the 1024 bytes at 16 * (kFaThreads * j + 64 * w), lane i
    // its 16 bytes at + 16 * i (the LDS address is the wave-uniform base plus
    // 16 * lane).
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    auto load_tile = [&](int kt, _Float16 *dst) {
        const _Float16 *src = tiles + static_cast<long long>(kt) * BUF;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int base = 8 * (kFaThreads * j + 64 * wv);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(src + base + 8 * lane),
                                             (__attribute__((address_space(3))) void *)(dst + base), 16, 0, 0);
        }
    };

    f32x16 o[RT][DT];
#pragma unroll
    for (int u = 0; u < RT; ++u)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[u][dt] = f32x16{};
    // Online softmax in log2 units against a reference m that is only raised
    // when a score exceeds it by more than 8 (weights stay <= 2^8, exact
    // enough in fp32 and in the fp16 split), so the accumulators are rarely
    // rescaled.
    float m[RT], l[RT];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
        m[u] = -INFINITY;
        l[u] = 0.0f;
    }
    const int kt0 = g_lo / kKeys, kt1 = (g_hi + kKeys - 1) / kKeys;
    // Tile kt lives in buffer kt & 1 (kt0 is odd when a window starts the
    // workgroup's keys past an odd tile).
    if (kt0 < kt1) load_tile(kt0, lds + (kt0 & 1) * BUF);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; ++kt) {
        // The other buffer was last read in the previous iteration, which
        // every wave finished before the barrier that ended it.
        if (kt + 1 < kt1) load_tile(kt + 1, lds + ((kt + 1) & 1) * BUF);
        const _Float16 *kh = lds + (kt & 1) * BUF;
        const _Float16 *kl = kh + kKeys * KS;
        const _Float16 *vh = kh + 2 * kKeys * KS;
        const _Float16 *vl = vh + D * kVtStride;
        const int k0 = kt * kKeys;
        if (k0 < w_hi && k0 + kKeys > w_lo) {
            // S^T tiles: accumulator r is key k0 + 8(r/4) + 4h + r%4 of row tw + 32u + nl.
            f32x16 s[RT];
#pragma unroll
            for (int u = 0; u < RT; ++u) s[u] = f32x16{};
#pragma unroll
            for (int st = 0; st < STEPS; ++st) {
                const half8 ah = *reinterpret_cast<const half8 *>(kh + nl * KS + 16 * st + 8 * h);
                const half8 al = *reinterpret_cast<const half8 *>(kl + nl * KS + 16 * st + 8 * h);
#pragma unroll
                for (int u = 0; u < RT; ++u) {
                    s[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qhf[u][st], s[u], 0, 0, 0);
                    s[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qhf[u][st], s[u], 0, 0, 0);
                    s[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qlf[u][st], s[u], 0, 0, 0);
                }
            }
            if (cap2 > 0.0f) {
#pragma unroll
                for (int u = 0; u < RT; ++u)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s[u][r] = cap2 * tanhf(s[u][r] / cap2);
            }
            if (!(k0 >= full_lo && k0 + kKeys <= full_hi)) {
#pragma unroll
                for (int u = 0; u < RT; ++u)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int kk = k0 + 8 * (r >> 2) + 4 * h + (r & 3);
                        if (kk < lo_t[u] || kk >= hi_t[u]) s[u][r] = -INFINITY;
                    }
            }
            float mx[RT];
            bool grow = false;
#pragma unroll
            for (int u = 0; u < RT; ++u) {
                float v = s[u][0];
#pragma unroll
                for (int r = 1; r < 16; ++r) v = fmaxf(v, s[u][r]);
                mx[u] = fmaxf(v, __shfl_xor(v, 32));
                grow = grow || mx[u] > m[u] + 8.0f;
            }
            if (__any(grow)) {
#pragma unroll
                for (int u = 0; u < RT; ++u) {
                    if (mx[u] > m[u] + 8.0f) {
                        const float alpha = __builtin_amdgcn_exp2f(m[u] - mx[u]);   // 0 while m is -inf
                        l[u] *= alpha;
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) o[u][dt] *= alpha;
                        m[u] = mx[u];
                    }
                }
            }
            // O^T += V^T P^T over the tile's keys in two MFMA steps of 16.
            // Lane half h supplies contraction entries e = 0..3 -> key
            // 16j + 4h + e and e = 4..7 -> key 16j + 8 + 4h + e - 4: the keys
            // of its score accumulators 8j .. 8j+7.
            half8 ph[RT][2], pl[RT][2];
#pragma unroll
            for (int u = 0; u < RT; ++u) {
                const float mref = m[u] == -INFINITY ? 0.0f : m[u];   // every score so far masked: weights 0
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float pv = __builtin_amdgcn_exp2f(s[u][r] - mref);
                    l[u] += pv;
                    _Float16 a, c;
                    split_half(pv, a, c);
                    ph[u][r >> 3][r & 7] = a;
                    pl[u][r >> 3][r & 7] = c;
                }
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const int off = (32 * dt + nl) * kVtStride + 16 * j + 4 * h;
                    const half4 h0 = *reinterpret_cast<const half4 *>(vh + off);
                    const half4 h1 = *reinterpret_cast<const half4 *>(vh + off + 8);
                    const half4 l0 = *reinterpret_cast<const half4 *>(vl + off);
                    const half4 l1 = *reinterpret_cast<const half4 *>(vl + off + 8);
                    const half8 ah = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                    const half8 al = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
#pragma unroll
                    for (int u = 0; u < RT; ++u) {
                        o[u][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ph[u][j], o[u][dt], 0, 0, 0);
                        o[u][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, ph[u][j], o[u][dt], 0, 0, 0);
                        o[u][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, pl[u][j], o[u][dt], 0, 0, 0);
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);               // this wave's copies of tile kt + 1 have landed
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < RT; ++u) {
        // The two lane halves hold partial sums of one row under one reference.
        const float lt = l[u] + __shfl_xor(l[u], 32);
        const int t = tw + 32 * u + nl;
        if (t < p.T) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            float *orow = p.out + b * p.q_b + t * p.q_t + head * p.q_h;
            // Accumulator r of tile dt is d = 32dt + 8(r/4) + 4h + r%4.
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<float4 *>(orow + 32 * dt + 8 * j + 4 * h) =
                        make_float4(o[u][dt][4 * j] * inv, o[u][dt][4 * j + 1] * inv, o[u][dt][4 * j + 2] * inv,
                                    o[u][dt][4 * j + 3] * inv);
        }
    }
}

// One wave per (b, t, head) query row, any D <= 256: scores of a chunk of
// up to kGenChunk keys in LDS (one key per lane at a time), then each lane
// accumulates its d = lane, lane + 64, ... over the chunk. fp32 throughout.
__global__ __launch_bounds__(64) void fa_generic_kernel(FaParams p, int D) {
    __shared__ float sc[kGenChunk];
    const int lane = threadIdx.x;
    long long idx = blockIdx.x;
    const int head = static_cast<int>(idx % p.H);
    idx /= p.H;
    const int t = static_cast<int>(idx % p.T);
    const int b = static_cast<int>(idx / p.T);
    const int kvh = head / p.G;
    const int hi = key_hi(p, t), lo = key_lo(p, hi);
    const float *qr = p.q + b * p.q_b + t * p.q_t + head * p.q_h;
    const float *kbase = p.k + b * p.k_b + kvh * p.k_h;
    const float *vbase = p.v + b * p.k_b + kvh * p.k_h;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    for (int c0 = lo; c0 < hi; c0 += kGenChunk) {
        const int n = min(kGenChunk, hi - c0);
        float mx = -INFINITY;
        for (int i = lane; i < n; i += 64) {
            const float *kr = kbase + static_cast<long long>(c0 + i) * p.k_s;
            float dot = 0.0f;
            for (int e = 0; e < D; ++e) dot = fmaf(qr[e], kr[e], dot);
            const float v = score_log2(dot * p.scale, p.soft_cap);
            sc[i] = v;
            mx = fmaxf(mx, v);
        }
        mx = wave_max(mx);
        const float mn = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.0f : exp2f(m - mn);
        __syncthreads();
        float ps = 0.0f;
        for (int i = lane; i < n; i += 64) {
            const float e = exp2f(sc[i] - mn);
            sc[i] = e;
            ps += e;
        }
        l = l * alpha + wave_sum(ps);
        m = mn;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < D) {
                float a = acc[j] * alpha;
                for (int i = 0; i < n; ++i) a = fmaf(sc[i], vbase[static_cast<long long>(c0 + i) * p.k_s + d], a);
                acc[j] = a;
            }
        }
        __syncthreads();
    }
    float *orow = p.out + b * p.q_b + t * p.q_t + head * p.q_h;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < D) orow[d] = acc[j] * inv;
    }
}

template <int D, int RT>
void launch_fa(int nqb, const FaParams &p0, hipStream_t s, const _Float16 *pk, int ntiles) {
    static bool lds_set = false;                 // the attribute is per kernel, per process
    if (!lds_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(fa_prefill_kernel<D, RT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(fa_lds_bytes<D>()));
        lds_set = true;
    }
    FaParams p = p0;
    p.nqb = nqb;
    const dim3 grid(static_cast<unsigned>(static_cast<long long>(nqb) * p.H * p.B)), block(kFaThreads);
    hipLaunchKernelGGL((fa_prefill_kernel<D, RT>), grid, block, fa_lds_bytes<D>(), s, p, pk, ntiles);
}

int enqueue_fa4(const void *out, const void *q, const void *k, const void *v, int B, int T, int S, int H, int Hkv,
                int D, float scale, int causal, float soft_cap, int window) {
    FaParams p{};
    p.q = static_cast<const float *>(q);
    p.k = static_cast<const float *>(k);
    p.v = static_cast<const float *>(v);
    p.out = static_cast<float *>(const_cast<void *>(out));
    p.q_h = D;
    p.q_t = static_cast<long long>(H) * D;
    p.q_b = p.q_t * T;
    p.k_h = D;
    p.k_s = static_cast<long long>(Hkv) * D;
    p.k_b = p.k_s * S;
    p.B = B;
    p.T = T;
    p.S = S;
    p.H = H;
    p.Hkv = Hkv;
    p.G = H / Hkv;
    p.scale = scale;
    p.soft_cap = soft_cap;
    p.causal = causal != 0;
    p.window = window > 0 ? window : 0;
    hipStream_t s = current_stream();
    const bool fast = (D == 64 || D == 128) && aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                      aligned(out, 16);
    if (fast) {
        // Two 32-row tiles per wave (one wave per SIMD) when that still gives
        // every CU four workgroups, whose uneven causal lengths then even
        // out; one tile (two waves per SIMD) otherwise.
        const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
        const int nqb2 = (T + 2 * kRowsWg - 1) / (2 * kRowsWg), nqb1 = (T + kRowsWg - 1) / kRowsWg;
        const bool two = static_cast<long long>(nqb2) * H * B >= 4LL * cus;
        const long long wgs = static_cast<long long>(two ? nqb2 : nqb1) * H * B;
        const int ntiles = (S + kKeys - 1) / kKeys;
        const long long packs = static_cast<long long>(B) * Hkv * ntiles;
        if (wgs > 0x7fffffffLL || packs > 0x7fffffffLL)
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "fa4_attention: grid too large");
        const size_t tile_bytes = D == 64 ? fa_tile_halves<64>() * 2 : fa_tile_halves<128>() * 2;
        _Float16 *pk = static_cast<_Float16 *>(stream_scratch(static_cast<size_t>(packs) * tile_bytes));
        if (!pk) return ALJABR_ROCM_ERR_BUFFER;
        if (D == 64) {
            hipLaunchKernelGGL(fa_pack_kernel<64>, dim3(static_cast<unsigned>(packs)), dim3(256), 0, s, p, pk, ntiles);
            if (two) launch_fa<64, 2>(nqb2, p, s, pk, ntiles);
            else launch_fa<64, 1>(nqb1, p, s, pk, ntiles);
        } else {
            hipLaunchKernelGGL(fa_pack_kernel<128>, dim3(static_cast<unsigned>(packs)), dim3(256), 0, s, p, pk, ntiles);
            if (two) launch_fa<128, 2>(nqb2, p, s, pk, ntiles);
            else launch_fa<128, 1>(nqb1, p, s, pk, ntiles);
        }
        return ALJABR_ROCM_OK;
    }
    if (D > 256) return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "fa4_attention: head size %d > 256", D);
    const long long rows = static_cast<long long>(B) * T * H;
    if (rows > 0x7fffffffLL) return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "fa4_attention: grid too large");
    hipLaunchKernelGGL(fa_generic_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), 0, s, p, D);
    return ALJABR_ROCM_OK;
}

}  // namespace


}  // namespace aljabr

using namespace aljabr;

namespace {

int fa4_checked(void *output, const void *query, const void *key, const void *value, int B, int T, int S, int H,
                int H_kv, int D, float scale, int is_causal, float soft_cap, int window) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(output && query && key && value, "fa4_attention: output, query, key and value must be non-null");
    ALJ_REQUIRE(B > 0 && T > 0 && S > 0 && H > 0 && H_kv > 0 && D > 0 && H % H_kv == 0,
                "fa4_attention expects Q/out [B,T,H,D], K/V [B,S,H_kv,D] with H divisible by H_kv");
    ALJ_REQUIRE(std::isfinite(scale) && std::isfinite(soft_cap), "fa4_attention: scale and soft_cap must be finite");
    ALJ_REQUIRE(static_cast<long long>(B) * T * H * D < (1LL << 40) && static_cast<long long>(B) * S * H_kv * D <
                                                                            (1LL << 40),
                "fa4_attention: tensors too large");
    const int rc = enqueue_fa4(output, query, key, value, B, T, S, H, H_kv, D, scale, is_causal, soft_cap, window);
    if (rc) return rc;
    return finish_launch("fa4_attention");
}

}  // namespace

extern "C" {

int aljabr_rocm_fa4_attention(void *output, const void *query, const void *key, const void *value, int B, int T,
                              int S, int H, int H_kv, int D, float scale, int is_causal, int use_bf16,
                              float soft_cap) {
    (void)use_bf16;   // computed to fp32 accuracy whatever the flag asks
    return fa4_checked(output, query, key, value, B, T, S, H, H_kv, D, scale, is_causal, soft_cap, 0);
}

int aljabr_rocm_fa4_attention_windowed(void *output, const void *query, const void *key, const void *value, int B,
                                       int T, int S, int H, int H_kv, int D, float scale, int is_causal,
                                       float soft_cap, int window) {
    return fa4_checked(output, query, key, value, B, T, S, H, H_kv, D, scale, is_causal, soft_cap, window);
}

int aljabr_rocm_fa4_sdpa_available(void) { return 1; }

int aljabr_rocm_fa4_bf16_available(void) { return 0; }

}  // extern "C"
