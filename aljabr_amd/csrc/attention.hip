// attention.hip - grouped-query attention over a KV cache on gfx950.
//
// Semantics follow CpuBackend.attentionGqa / computeAttentionGroup
// (backend/cpu/aljabr-backend-cpu/.../CpuBackend.java:1546-1748): per query
// row, online softmax over the visible keys; bottom-right causal alignment
// (key limit = Sk - Sq + qi + 1); an additive mask entry of -inf skips the key;
// a row with no visible key yields 0.
//
// Split-K design (head_dim 64 or 128). Work item = (batch, kv head, query
// row); its key range is cut into `splits` chunks, one workgroup each. A
// workgroup serves all G = Hq/Hkv query heads of its KV head, so every K/V
// byte is read once per query row. Inside a workgroup, a key row of D fp16
// values is read by D/8 lanes (16 bytes each); the wave's lane groups walk
// interleaved keys in tiles of 4 (2 when a chunk is one trip), keep (max,
// sum, o[8]) per head in registers, and reduce q.k across the group's lanes
// with DPP. A wave's group states are folded by lane shuffles and the wave
// states merged through LDS; with one split the workgroup writes the
// normalised output, otherwise (m, l, o) partials go to scratch and a merge
// kernel combines splits. Scores use exp2 with log2(e) folded into the query.
#include <cmath>
#include <cstdlib>
#include <mutex>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {

namespace {

constexpr float kLog2e = 1.4426950408889634f;

// 2^x with one v_exp_f32 (exp2f adds a denormal-range fix-up of five more
// instructions). Every use is a softmax weight relative to a running maximum
// (x <= 0): a result below 2^-126 flushes to 0, a weight below 1e-38 of the
// largest one, and 2^-inf = 0.
__device__ __forceinline__ float exp2_w(float x) { return __builtin_amdgcn_exp2f(x); }

template <int LPK>
__device__ __forceinline__ float group_sum(float v) {
    // Sum over the LPK lanes of a key group (LPK = 8 or 16, aligned groups).
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    if constexpr (LPK == 16) v += dpp_f32<0x140>(v);
    return v;
}

// Raw K/V slice of one key as loaded (8 fp16 or 8 fp32 values).
template <bool F16> struct KvRaw;
template <> struct KvRaw<true> { uint4 u; };
template <> struct KvRaw<false> { float4 a, b; };

template <bool F16>
__device__ __forceinline__ KvRaw<F16> load_raw(const void *base, long long idx) {
    KvRaw<F16> r;
    if constexpr (F16) {
        r.u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + idx);
    } else {
        r.a = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx);
        r.b = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx + 4);
    }
    return r;
}

// All-zero bits (+0.0 values) unless `keep`: masks a raw K/V slice before
// conversion, so the conversions can fold into the FMAs that read them.
template <bool F16>
__device__ __forceinline__ KvRaw<F16> masked(KvRaw<F16> x, bool keep) {
    const uint32_t k = keep ? 0xffffffffu : 0u;
    if constexpr (F16) {
        x.u.x &= k; x.u.y &= k; x.u.z &= k; x.u.w &= k;
    } else {
        x.a = make_float4(__uint_as_float(__float_as_uint(x.a.x) & k), __uint_as_float(__float_as_uint(x.a.y) & k),
                          __uint_as_float(__float_as_uint(x.a.z) & k), __uint_as_float(__float_as_uint(x.a.w) & k));
        x.b = make_float4(__uint_as_float(__float_as_uint(x.b.x) & k), __uint_as_float(__float_as_uint(x.b.y) & k),
                          __uint_as_float(__float_as_uint(x.b.z) & k), __uint_as_float(__float_as_uint(x.b.w) & k));
    }
    return x;
}

template <bool F16>
__device__ __forceinline__ void raw_to_f32(const KvRaw<F16> &x, float (&r)[8]) {
    if constexpr (F16) {
        const uint32_t w[4] = {x.u.x, x.u.y, x.u.z, x.u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
            r[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
        }
    } else {
        r[0] = x.a.x; r[1] = x.a.y; r[2] = x.a.z; r[3] = x.a.w;
        r[4] = x.b.x; r[5] = x.b.y; r[6] = x.b.z; r[7] = x.b.w;
    }
}

template <bool F16>
__device__ __forceinline__ void load8(const void *base, long long idx, float (&r)[8]) {
    if constexpr (F16) {
        const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + idx);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
            r[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
        }
    } else {
        const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx);
        const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx + 4);
        r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
        r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
    }
}

// grid: x = split, y = kv head * Sq + query row, z = batch. WAVES*64 threads.
// Visible key range [lo, hi) of query row qi for a sequence of sk keys.
__device__ __forceinline__ void key_range(const AttnParams &p, int sk, int qi, int &lo, int &hi) {
    if (p.paged_bounds) {
        // MTLC/aljabr_metal_attention.m:146-160,192-200.
        int qpos = p.query_start + qi;
        if (p.causal && p.window <= 0 && p.query_start == 0 && sk >= p.Sq) qpos = sk - p.Sq + qi;
        int upper = p.causal ? qpos : sk - 1;
        if (upper >= sk) upper = sk - 1;
        int lower = p.window > 0 ? qpos - p.window + 1 : 0;
        if (lower < 0) lower = 0;
        lo = lower;
        hi = upper + 1;
    } else {
        // CPU/CpuBackend.java:1690-1700: bottom-right causal limit.
        lo = 0;
        hi = sk;
        if (p.causal) {
            const int c = sk - p.Sq + qi + 1;
            hi = c < sk ? c : sk;
        }
    }
}

// Merge the split partials of one query row with NTH threads: D/4 lanes take
// one split's o as float4s, so NTH/(D/4) splits are read at once; each lane
// group folds its splits (in split order) with online rescaling, and the
// groups are combined through `st` ([NTH/(D/4)][D + 2] floats of LDS).
template <int D, int NTH>
__device__ __forceinline__ void merge_row(const float *__restrict__ part_o, const float *__restrict__ part_ml,
                                          float *out_base, int splits, long long row, int Sq, int Hq, int q_sb,
                                          int q_sh, int q_sq, float norm_eps, float *st, uint16_t *xpack = nullptr) {
    constexpr int LPS = D / 4;          // lanes per split
    constexpr int SG = NTH / LPS;       // splits in flight
    const int qi = static_cast<int>(row % Sq);
    const int h = static_cast<int>((row / Sq) % Hq);
    const int bb = static_cast<int>(row / (static_cast<long long>(Sq) * Hq));
    float *out = out_base + static_cast<long long>(bb) * q_sb + static_cast<long long>(h) * q_sh +
                 static_cast<long long>(qi) * q_sq;
    const int sg = threadIdx.x / LPS, j = threadIdx.x % LPS;
    const float *po = part_o + row * splits * D;
    const float *pm = part_ml + row * splits * 2;
    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // Eight splits per trip with all their loads issued before any is used
    // (one memory round trip per trip instead of one per split).
    constexpr int U = 8;
    for (int s0 = sg; s0 < splits; s0 += U * SG) {
        float ms[U], ls[U];
        float4 os[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u * SG;
            const int sc = s < splits ? s : sg;                 // in-range row, ignored below
            ms[u] = pm[2 * sc];
            ls[u] = pm[2 * sc + 1];
            os[u] = *reinterpret_cast<const float4 *>(po + sc * D + 4 * j);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + u * SG >= splits) break;
            const float mn = fmaxf(m, ms[u]);
            if (mn == -INFINITY) continue;
            const float a = m == -INFINITY ? 0.0f : exp2_w(m - mn);
            const float b = ms[u] == -INFINITY ? 0.0f : exp2_w(ms[u] - mn);
            l = fmaf(l, a, ls[u] * b);
            o.x = fmaf(o.x, a, os[u].x * b);
            o.y = fmaf(o.y, a, os[u].y * b);
            o.z = fmaf(o.z, a, os[u].z * b);
            o.w = fmaf(o.w, a, os[u].w * b);
            m = mn;
        }
    }
    float *my = st + sg * (D + 2);
    my[4 * j] = o.x;
    my[4 * j + 1] = o.y;
    my[4 * j + 2] = o.z;
    my[4 * j + 3] = o.w;
    if (j == 0) {
        my[D] = m;
        my[D + 1] = l;
    }
    __syncthreads();
    for (int dd = threadIdx.x; dd < D; dd += NTH) {
        float M = -INFINITY;
#pragma unroll
        for (int g = 0; g < SG; ++g) M = fmaxf(M, st[g * (D + 2) + D]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int g = 0; g < SG; ++g) {
                const float mg = st[g * (D + 2) + D];
                if (mg == -INFINITY) continue;
                const float w = exp2_w(mg - M);
                L = fmaf(st[g * (D + 2) + D + 1], w, L);
                O = fmaf(st[g * (D + 2) + dd], w, O);
            }
        }
        const float val = L == 0.0f ? 0.0f : O / (L + norm_eps);
        out[dd] = val;
        if (xpack) xpack[xpack_index(bb, h * D + dd, Hq * D)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(val));
    }
    __syncthreads();                    // `st` is free again
}

// Merge split partials: one 256-thread workgroup per query row. Every
// argument is a scalar (preloaded into SGPRs at wave launch): the partial
// loads go out without an argument read first.
template <int D>
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ part_o,
                                                        const float *__restrict__ part_ml, float *out, int splits,
                                                        int Sq, int Hq, int q_sb, int q_sh, int q_sq, float norm_eps,
                                                        uint16_t *xpack) {
    __shared__ float st[(256 / (D / 4)) * (D + 2)];
    merge_row<D, 256>(part_o, part_ml, out, splits, blockIdx.x, Sq, Hq, q_sb, q_sh, q_sq, norm_eps, st, xpack);
}

// KT keys per group per trip (the tile): 4, or 2 where a workgroup's chunk
// is one trip of 2-key tiles (every group busy, half the serial work per
// lane).
// The arguments the first K/V and q loads need lead as scalars (preloaded
// into SGPRs at wave launch, 14 dwords): the caches, q, the lengths, the
// row stride cap (= the rows in memory: callers of the contiguous path pass
// cap == Sk), Sq | Hkv << 16, the chunk and q's element strides (32-bit).
template <int D, int G, bool F16, int WAVES, bool PAGED, int KT>
__global__ __launch_bounds__(WAVES * 64) void attn_split_kernel(const void *kcache, const void *vcache,
                                                                const float *q, const int *kv_len, int cap,
                                                                int sq_hkv, int chunk, int q_sb, int q_sh, int q_sq,
                                                                AttnParams p, int splits, float *__restrict__ part_o,
                                                                float *__restrict__ part_ml) {
    const int Sq = sq_hkv & 0xffff, Hkv = sq_hkv >> 16;
    constexpr int LPK = D / 8;                 // lanes per key row
    constexpr int GPW = 64 / LPK;              // key groups per wave
    constexpr int NG = GPW * WAVES;            // key groups per workgroup
    extern __shared__ float smem[];            // [WAVES][G][D + 2]

    const int split = blockIdx.x;
    const int kvh = blockIdx.y / Sq;
    const int qi = blockIdx.y % Sq;
    const int b = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int grp = wave * GPW + lane / LPK;   // key group in workgroup
    const int sub = lane % LPK;                // 8-dim slice of the row

    const int k_begin = split * chunk;
    // Element offset of key row `key` (this lane's 8-value slice).
    const long long head_base = (static_cast<long long>(b) * Hkv + kvh) * cap * D + sub * 8;
    const int *btab = PAGED ? p.block_table + static_cast<long long>(b) * p.max_blocks : nullptr;
    auto row_at = [&](int key) -> long long {
        if constexpr (PAGED) {
            const int blk = key / p.block_size;
            const int phys = max(btab[blk], 0);
            return ((static_cast<long long>(phys) * Hkv + kvh) * p.block_size + (key - blk * p.block_size)) * D +
                   sub * 8;
        } else {
            return head_base + static_cast<long long>(key) * D;
        }
    };
    KvRaw<F16> kn[KT], vn[KT];
    int mem_end;                                 // keys below this are rows that exist
    auto issue = [&](int tbase) {
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const int key = tbase + t;
            const long long r = row_at(key < mem_end ? key : k_begin);
            kn[t] = load_raw<F16>(kcache, r);
            vn[t] = load_raw<F16>(vcache, r);
        }
    };
    // Query slices, loaded before the length is read (they do not depend on
    // it) and scaled below.
    float4 qa[G], qc[G];
    auto load_q = [&]() {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int h = kvh * G + g;
            const float *qp = q + static_cast<long long>(b) * q_sb + static_cast<long long>(h) * q_sh +
                              static_cast<long long>(qi) * q_sq + sub * 8;
            qa[g] = *reinterpret_cast<const float4 *>(qp);
            qc[g] = *reinterpret_cast<const float4 *>(qp + 4);
        }
    };
    int sk;
    if constexpr (PAGED) {
        // Blocks past the sequence's length may not exist: read the length
        // first, and a split past it loads nothing (clamped keys fall back
        // to k_begin, which must then be a row of the sequence).
        load_q();
        sk = max(kv_len[b], 0);
        mem_end = min(k_begin + chunk, sk);
        if (k_begin < sk) issue(k_begin + grp * KT);
    } else {
        // Rows [k_begin, mem_end) exist in memory whatever the visible length,
        // so the first tile's loads go out before kv_len has arrived.
        mem_end = min(k_begin + chunk, cap);
        issue(k_begin + grp * KT);
        load_q();
        sk = kv_len ? min(max(kv_len[b], 0), cap) : cap;          // never past the cache
    }
    int k_lo, k_hi;
    key_range(p, sk, qi, k_lo, k_hi);
    int k_end = k_begin + chunk;
    if (k_end > k_hi) k_end = k_hi;

    // Query slices, pre-scaled so that exp2(q.k) == exp(score).
    float qv[G][8];
    const float qs = p.scale * kLog2e;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float4 a = qa[g], c = qc[g];
        qv[g][0] = a.x * qs; qv[g][1] = a.y * qs; qv[g][2] = a.z * qs; qv[g][3] = a.w * qs;
        qv[g][4] = c.x * qs; qv[g][5] = c.y * qs; qv[g][6] = c.z * qs; qv[g][7] = c.w * qs;
    }

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = 0.0f;
    }

    const float *mrow = p.mask ? p.mask + static_cast<long long>(qi) * p.Sk : nullptr;

    // Software pipeline: the next tile's K/V rows are loaded while this one
    // is computed. Only a group with another trip loads one: the tile is the
    // only load in flight at the loop head, so the wait there is the one the
    // tile needs anyway, and a group's last trip leaves nothing in flight
    // (a prefetch past the end would be waited for before the merge).
    for (int t0 = k_begin + grp * KT; t0 < k_end; t0 += NG * KT) {
        float kr[KT][8], vr[KT][8];
        bool valid[KT];
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            valid[t] = t0 + t < k_end && (!PAGED || t0 + t >= k_lo);   // only the paged rule has a lower bound
            raw_to_f32<F16>(kn[t], kr[t]);
            // Rows past the visible keys may hold anything (the first tile is
            // loaded before the length is known, and cache rows beyond a
            // sequence's length were never written): their values must not
            // reach the sums, where 0 * NaN would still be NaN. Masked as raw
            // bits (four selects per key for fp16), so the conversions fold
            // into the P.V FMAs.
            raw_to_f32<F16>(masked<F16>(vn[t], valid[t]), vr[t]);
        }
        if (t0 + NG * KT < k_end) issue(t0 + NG * KT);
        float add[KT];
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            add[t] = 0.0f;
            if (mrow && valid[t]) add[t] = mrow[t0 + t] * kLog2e;
            if (!valid[t]) add[t] = -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s[KT];
            float tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d = fmaf(qv[g][i], kr[t][i], d);
                d = group_sum<LPK>(d);
                if (PAGED && p.soft_cap > 0.0f) {
                    // d = score * log2(e): cap the score, then back to base 2.
                    const float cap = p.soft_cap;
                    d = cap * tanhf(d / (kLog2e * cap)) * kLog2e;
                }
                s[t] = valid[t] ? d + add[t] : -INFINITY;
                tmax = fmaxf(tmax, s[t]);
            }
            const float mn = fmaxf(m[g], tmax);
            if (mn == -INFINITY) continue;             // nothing visible yet
            const float alpha = exp2_w(m[g] - mn);   // mn is finite here: m = -inf gives 0
            float psum = 0.0f;
            float pr[KT];
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                pr[t] = exp2_w(s[t] - mn);            // s = -inf (masked) gives 0
                psum += pr[t];
            }
            l[g] = fmaf(l[g], alpha, psum);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float acc = o[g][i] * alpha;
#pragma unroll
                for (int t = 0; t < KT; ++t) acc = fmaf(pr[t], vr[t][i], acc);
                o[g][i] = acc;
            }
            m[g] = mn;
        }
    }

    // Fold the wave's key groups into one state: lanes `off` apart hold the
    // same dims of two groups (m and l are uniform within a group); an empty
    // state (m = -inf, l = o = 0) weighs 0.
#pragma unroll
    for (int off = 32; off >= LPK; off >>= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float m2 = __shfl_xor(m[g], off);
            const float l2 = __shfl_xor(l[g], off);
            float o2[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o2[i] = __shfl_xor(o[g][i], off);
            const float mn = fmaxf(m[g], m2);
            const float a = m[g] == -INFINITY ? 0.0f : exp2_w(m[g] - mn);
            const float c = m2 == -INFINITY ? 0.0f : exp2_w(m2 - mn);
            l[g] = fmaf(l[g], a, l2 * c);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[g][i] = fmaf(o[g][i], a, o2[i] * c);
            m[g] = mn;
        }
    }

    // Publish wave states: smem[wave][g][0..D) = o, [D] = m, [D+1] = l.
    if (lane < LPK) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float *st = smem + (wave * G + g) * (D + 2);
#pragma unroll
            for (int i = 0; i < 8; ++i) st[sub * 8 + i] = o[g][i];
            if (sub == 0) {
                st[D] = m[g];
                st[D + 1] = l[g];
            }
        }
    }
    __syncthreads();

    // Merge the WAVES wave states; one thread per (head, dim). All states
    // are read before any is used (the reads overlap instead of queueing
    // behind each other).
    for (int idx = threadIdx.x; idx < G * D; idx += WAVES * 64) {
        const int g = idx / D, dd = idx % D;
        float mg[WAVES], lg[WAVES], og[WAVES];
#pragma unroll
        for (int gr = 0; gr < WAVES; ++gr) {
            const float *st = smem + (gr * G + g) * (D + 2);
            mg[gr] = st[D];
            lg[gr] = st[D + 1];
            og[gr] = st[dd];
        }
        float M = -INFINITY;
#pragma unroll
        for (int gr = 0; gr < WAVES; ++gr) M = fmaxf(M, mg[gr]);
        float L = 0.0f, O = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int gr = 0; gr < WAVES; ++gr) {
                const float w = mg[gr] == -INFINITY ? 0.0f : exp2_w(mg[gr] - M);
                L = fmaf(lg[gr], w, L);
                O = fmaf(og[gr], w, O);
            }
        }
        const int h = kvh * G + g;
        const long long row = (static_cast<long long>(b) * p.Hq + h) * p.Sq + qi;
        if (splits == 1) {
            const float val = L == 0.0f ? 0.0f : O / (L + p.norm_eps);
            p.out[b * p.q_sb + h * p.q_sh + qi * p.q_sq + dd] = val;
            if (p.xpack)
                p.xpack[xpack_index(b, h * D + dd, p.Hq * D)] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(val));
        } else {
            part_o[(row * splits + split) * D + dd] = O;
            if (dd == 0) {
                part_ml[(row * splits + split) * 2] = M;
                part_ml[(row * splits + split) * 2 + 1] = L;
            }
        }
    }
}

// Any head_dim: one thread per (batch, query head, query row, output dim).
// Each thread runs computeAttentionGroup's loop for its own dimension,
// including the double-precision denominator and weighted value.
template <bool F16>
__device__ __forceinline__ float kv_at(const void *base, long long i) {
    if constexpr (F16) return f16_bits_to_f32(static_cast<const uint16_t *>(base)[i]);
    else return static_cast<const float *>(base)[i];
}

template <bool F16>
__global__ __launch_bounds__(64) void attn_generic_kernel(AttnParams p) {
    const long long tid = static_cast<long long>(blockIdx.x) * 64 + threadIdx.x;
    const int D = p.D;
    const long long total = static_cast<long long>(p.B) * p.Hq * p.Sq * D;
    if (tid >= total) return;
    const int j = static_cast<int>(tid % D);
    const long long idx = tid / D;   // query row (b * Hq + h) * Sq + qi
    const int qi = static_cast<int>(idx % p.Sq);
    const int h = static_cast<int>((idx / p.Sq) % p.Hq);
    const int b = static_cast<int>(idx / (static_cast<long long>(p.Sq) * p.Hq));
    const int kvh = h / (p.Hq / p.Hkv);
    const int sk = p.block_table ? max(p.kv_len[b], 0)
                                 : (p.kv_len ? min(max(p.kv_len[b], 0), p.cap) : p.Sk);   // never past the cache
    int lo, hi;
    key_range(p, sk, qi, lo, hi);
    const float *qr = p.q + b * p.q_sb + h * p.q_sh + qi * p.q_sq;
    auto row_at = [&](int ki) -> long long {
        if (p.block_table) {
            const int blk = ki / p.block_size;
            const int phys = max(p.block_table[static_cast<long long>(b) * p.max_blocks + blk], 0);
            return ((static_cast<long long>(phys) * p.Hkv + kvh) * p.block_size + (ki - blk * p.block_size)) * D;
        }
        return ((static_cast<long long>(b) * p.Hkv + kvh) * p.cap + ki) * D;
    };
    float running = -INFINITY;
    double den = 0.0, weighted = 0.0;
    for (int ki = lo; ki < hi; ++ki) {
        const float add = p.mask ? p.mask[static_cast<long long>(qi) * p.Sk + ki] : 0.0f;
        if (add == -INFINITY) continue;
        const long long kb = row_at(ki);
        float dot = 0.0f;
        for (int e = 0; e < D; ++e) dot = fmaf(qr[e], kv_at<F16>(p.k, kb + e), dot);
        float score = dot * p.scale;
        if (p.soft_cap > 0.0f) score = p.soft_cap * tanhf(score / p.soft_cap);
        score += add;
        float next;
        double prev_s, cur_s;
        if (isfinite(score)) {
            if (score > running) {
                prev_s = exp(static_cast<double>(running - score));
                cur_s = 1.0;
                next = score;
            } else {
                prev_s = 1.0;
                cur_s = exp(static_cast<double>(score - running));
                next = running;
            }
        } else {
            next = fmaxf(running, score);
            prev_s = running == -INFINITY ? 0.0 : exp(static_cast<double>(running - next));
            cur_s = exp(static_cast<double>(score - next));
        }
        den = den * prev_s + cur_s;
        weighted = weighted * prev_s + cur_s * kv_at<F16>(p.v, kb + j);
        running = next;
    }
    p.out[b * p.q_sb + h * p.q_sh + qi * p.q_sq + j] =
        den == 0.0 ? 0.0f : static_cast<float>(weighted / (den + static_cast<double>(p.norm_eps)));
}

__global__ void mask_check_kernel(const float *__restrict__ mask, long long n, int *__restrict__ bad) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        const float v = mask[i];
        if (v != v || v == INFINITY) atomicOr(bad, 1);
    }
}

__global__ void zero_i32_kernel(int *p) { *p = 0; }

// WIDE: 8-wave workgroups (4 with G = 8) for grids of about one workgroup
// per CU; 4-wave ones (2) otherwise.
template <int D, int G, bool F16, bool PAGED, bool WIDE>
int launch_split(const AttnParams &p, int splits, int chunk, float *part, hipStream_t s) {
    constexpr int WAVES = WIDE ? ((G <= 4) ? 8 : 4) : ((G <= 4) ? 4 : 2);
    constexpr int NG = (64 / (D / 8)) * WAVES;    // key groups per workgroup
    const size_t lds = static_cast<size_t>(WAVES) * G * (D + 2) * sizeof(float);
    static_assert(static_cast<size_t>(WAVES) * G * (D + 2) * sizeof(float) <= 65536, "static LDS limit");
    const dim3 grid(splits, p.Hkv * p.Sq, p.B);
    const long long rows = static_cast<long long>(p.B) * p.Hq * p.Sq;
    // Partials: o as [rows][splits][D], then (m, l) as [rows][splits][2].
    float *part_o = part;
    float *part_ml = part ? part + rows * splits * D : nullptr;
    const int sq_hkv = p.Sq | (p.Hkv << 16);
    const int qsb = static_cast<int>(p.q_sb), qsh = static_cast<int>(p.q_sh), qsq = static_cast<int>(p.q_sq);
    if (WIDE && chunk <= 2 * NG)
        hipLaunchKernelGGL((attn_split_kernel<D, G, F16, WAVES, PAGED, 2>), grid, dim3(WAVES * 64), lds, s, p.k, p.v,
                           p.q, p.kv_len, p.cap, sq_hkv, chunk, qsb, qsh, qsq, p, splits, part_o, part_ml);
    else
        hipLaunchKernelGGL((attn_split_kernel<D, G, F16, WAVES, PAGED, 4>), grid, dim3(WAVES * 64), lds, s, p.k, p.v,
                           p.q, p.kv_len, p.cap, sq_hkv, chunk, qsb, qsh, qsq, p, splits, part_o, part_ml);
    if (splits > 1)
        hipLaunchKernelGGL((attn_merge_kernel<D>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, part_o,
                           part_ml, p.out, splits, p.Sq, p.Hq, qsb, qsh, qsq, p.norm_eps, p.xpack);
    return ALJABR_ROCM_OK;
}

template <int D, bool F16, bool PAGED, bool WIDE>
int launch_g(const AttnParams &p, int G, int splits, int chunk, float *part, hipStream_t s) {
    switch (G) {
    case 1: return launch_split<D, 1, F16, PAGED, WIDE>(p, splits, chunk, part, s);
    case 2: return launch_split<D, 2, F16, PAGED, WIDE>(p, splits, chunk, part, s);
    case 4: return launch_split<D, 4, F16, PAGED, WIDE>(p, splits, chunk, part, s);
    case 8: return launch_split<D, 8, F16, PAGED, WIDE>(p, splits, chunk, part, s);
    default: return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "no split attention kernel for %d query heads per KV head", G);
    }
}

template <int D, bool F16>
int launch_paged(const AttnParams &p, int G, int splits, int chunk, float *part, bool wide, hipStream_t s) {
    if (wide)
        return p.block_table ? launch_g<D, F16, true, true>(p, G, splits, chunk, part, s)
                             : launch_g<D, F16, false, true>(p, G, splits, chunk, part, s);
    return p.block_table ? launch_g<D, F16, true, false>(p, G, splits, chunk, part, s)
                         : launch_g<D, F16, false, false>(p, G, splits, chunk, part, s);
}

}  // namespace

// Chunks hold at least 64 keys (rounded to 16), so there are at most
// ceil(keys / 64) + 1 splits.
size_t attention_scratch_bytes(int B, int Hq, int Sq, int D, int keys) {
    const size_t splits = static_cast<size_t>((keys + 63) / 64) + 1;
    return static_cast<size_t>(B) * Hq * Sq * splits * (D + 2) * sizeof(float);
}

// Enqueue attention (no sync). Chooses the split-K kernels for D in {64,128}
// with G in {1,2,4,8} and 16-byte aligned rows, the generic kernel otherwise.
int enqueue_attention(const AttnParams &p_in) {
    hipStream_t s = current_stream();
    AttnParams p = p_in;
    if (p.q_sq == 0) {                           // default layout [B][Hq][Sq][D]
        p.q_sq = p.D;
        p.q_sh = static_cast<long long>(p.Sq) * p.D;
        p.q_sb = static_cast<long long>(p.Hq) * p.Sq * p.D;
    }
    const int G = p.Hq / p.Hkv;
    // The split kernel takes Sq and Hkv packed in one word, q's strides as
    // 32-bit values and, for contiguous caches, cap as the rows in memory.
    const bool fast = (p.D == 64 || p.D == 128) && (G == 1 || G == 2 || G == 4 || G == 8) && aligned(p.q, 16) &&
                      aligned(p.out, 16) && aligned(p.k, 16) && aligned(p.v, 16) && p.q_sq % 4 == 0 &&
                      p.q_sh % 4 == 0 && p.q_sb % 4 == 0 && p.Sq <= 0xffff && p.Hkv <= 0x7fff &&
                      p.q_sb <= 0x7fffffffLL && p.q_sh <= 0x7fffffffLL && p.q_sq <= 0x7fffffffLL &&
                      (p.block_table || p.cap == p.Sk);
    if (p.xpack && (!fast || p.Sq != 1 || p.q_sh != p.D || p.q_sb != static_cast<long long>(p.Hq) * p.D ||
                    (p.Hq * p.D) % 64 != 0 || !aligned(p.xpack, 16)))
        return ALJABR_ROCM_ERR_UNSUPPORTED;
    if (!fast) {
        const long long n = static_cast<long long>(p.B) * p.Hq * p.Sq * p.D;
        const dim3 grid(static_cast<unsigned>((n + 63) / 64));
        if (p.kv_f16)
            hipLaunchKernelGGL(attn_generic_kernel<true>, grid, dim3(64), 0, s, p);
        else
            hipLaunchKernelGGL(attn_generic_kernel<false>, grid, dim3(64), 0, s, p);
        return ALJABR_ROCM_OK;
    }
    // Chunks of >= 64 keys. With at least two (sequence, KV head, query
    // row) items per CU: 4-wave workgroups, enough splits to cover the CUs
    // twice. With fewer: 8-wave workgroups, enough splits to cover them once
    // (measured on MI355X: batch 32 x 8 KV heads at 2048 keys 60.9 -> 56.6 us,
    // one split and no merge launch; batch 1 at 4096 keys 18.3 -> 16.8 us;
    // batch 64 was faster with the 4-wave shape).
    const long long items = static_cast<long long>(p.B) * p.Hkv * p.Sq;
    const int keys = p.block_table ? p.max_blocks * p.block_size : (p.kv_len ? p.cap : p.Sk);
    const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const bool wide = items < 2LL * cus;
    const int per_cu = wide ? 1 : 2;
    long long want = (static_cast<long long>(per_cu) * cus + items - 1) / items;
    const long long max_splits = (keys + 63) / 64;
    if (want > max_splits) want = max_splits;
    if (want < 1) want = 1;
    const size_t split_bytes = static_cast<size_t>(p.B) * p.Hq * p.Sq * (p.D + 2) * sizeof(float);
    if (p.scratch_only) {
        // Partials only in the caller's buffer: as many splits as it holds.
        const long long fit = p.scratch ? static_cast<long long>(p.scratch_bytes / split_bytes) : 0;
        if (want > fit) want = fit < 2 ? 1 : fit;
    }
    int splits = static_cast<int>(want);
    int chunk = (keys + splits - 1) / splits;
    chunk = (chunk + 15) & ~15;
    splits = (keys + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
    float *part = nullptr;
    if (splits > 1) {
        const size_t bytes = static_cast<size_t>(splits) * split_bytes;
        if (p.scratch && bytes <= p.scratch_bytes) part = p.scratch;
        else if (!p.scratch_only) part = static_cast<float *>(stream_scratch(bytes));
        if (!part) return p.scratch_only ? fail(ALJABR_ROCM_ERR_BUFFER, "attention: split partials exceed the caller's scratch")
                                         : ALJABR_ROCM_ERR_BUFFER;
    }
    if (p.D == 64)
        return p.kv_f16 ? launch_paged<64, true>(p, G, splits, chunk, part, wide, s)
                        : launch_paged<64, false>(p, G, splits, chunk, part, wide, s);
    return p.kv_f16 ? launch_paged<128, true>(p, G, splits, chunk, part, wide, s)
                    : launch_paged<128, false>(p, G, splits, chunk, part, wide, s);
}

}  // namespace aljabr

using namespace aljabr;

extern "C" int aljabr_rocm_attention_gqa(void *out, const void *Q, const void *K, const void *V, const void *mask,
                                         int B, int Hq, int Hkv, int Sq, int Sk, int D, int kvType, float scale,
                                         int causal) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(out && Q && K && V, "out, Q, K and V must be non-null device pointers");
    ALJ_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Sq > 0 && Sk > 0 && D > 0 && Hq % Hkv == 0,
                "GQA expects Q[B,Hq,Sq,D], K/V[B,Hkv,Sk,D] with Hq divisible by Hkv");
    if (kvType != ALJABR_ROCM_TYPE_F32 && kvType != ALJABR_ROCM_TYPE_F16)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "attention: K/V type %d is not F32 or F16", kvType);
    hipStream_t s = current_stream();
    if (mask) {
        // CpuBackend.validateAttentionMask: NaN or +inf anywhere is rejected.
        int *flag = static_cast<int *>(stream_scratch(sizeof(int)));
        if (!flag) return ALJABR_ROCM_ERR_BUFFER;
        const long long n = static_cast<long long>(Sq) * Sk;
        hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(1), 0, s, flag);
        hipLaunchKernelGGL(mask_check_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                           static_cast<const float *>(mask), n, flag);
        int bad = 0;
        hipError_t e = hipMemcpyAsync(&bad, flag, sizeof(int), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "attention mask check: %s", hipGetErrorString(e));
        if (bad) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "attention mask values must not be NaN or positive infinity");
    }
    AttnParams p{};
    p.out = static_cast<float *>(out);
    p.q = static_cast<const float *>(Q);
    p.k = K;
    p.v = V;
    p.mask = static_cast<const float *>(mask);
    p.kv_len = nullptr;
    p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Sq = Sq; p.Sk = Sk; p.D = D; p.cap = Sk;
    p.scale = scale > 0.0f ? scale : static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
    p.causal = causal != 0;
    p.kv_f16 = kvType == ALJABR_ROCM_TYPE_F16;
    int rc = enqueue_attention(p);
    if (rc) return rc;
    return finish_launch("attention_gqa");
}

// ---- allocation-free attention ---------------------------------------------
//
// aljabr_rocm_attention_gqa_noalloc keeps its split partials in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the
// process ends (kNoAllocSlots slots of kNoAllocSlotBytes each). Host code
// never passes the array's name to a kernel: it is a host-side stand-in, not
// a device address. The device address comes from hipGetSymbolAddress, once
// per device, with that device current, and is kept per device.
//
// Each slot belongs to one stream at a time, so calls on different streams
// never share partials: calls on one stream are ordered by the stream, and
// up to kNoAllocSlots streams per GPU run concurrently. A further stream
// takes the least recently used slot after the device has drained (so the
// slot's previous stream has finished with it). The slot is chosen and the
// work enqueued under one lock. Every slot a call reads was written by the
// same call (the split kernel writes every split's partials before the merge
// reads them), so nothing needs clearing.
namespace {

constexpr int kNoAllocSlots = 4;
constexpr size_t kNoAllocSlotBytes = size_t(8) << 20;      // 8 MiB per slot, 32 MiB per GPU
static __device__ __align__(256) float scratch[kNoAllocSlots * kNoAllocSlotBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
struct NoAllocDevice {
    float *base = nullptr;                  // device address of `scratch` on this device
    hipStream_t owner[kNoAllocSlots] = {};
    bool taken[kNoAllocSlots] = {};
    uint64_t last_use[kNoAllocSlots] = {};
    uint64_t clock = 0;
};
std::mutex g_scratch_mu;                    // guards g_noalloc and spans slot choice + enqueue
NoAllocDevice g_noalloc[kMaxDevices];

// The slot of stream `s` on the current device (caller holds g_scratch_mu).
int noalloc_slot(hipStream_t s, float **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(ALJABR_ROCM_ERR_DEVICE, "device ordinal %d out of range", dev);
    NoAllocDevice &d = g_noalloc[dev];
    if (!d.base) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(ALJABR_ROCM_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        d.base = static_cast<float *>(ptr);
    }
    int pick = -1;
    for (int i = 0; i < kNoAllocSlots && pick < 0; ++i)
        if (d.taken[i] && d.owner[i] == s) pick = i;
    for (int i = 0; i < kNoAllocSlots && pick < 0; ++i)
        if (!d.taken[i]) pick = i;
    if (pick < 0) {
        pick = 0;
        for (int i = 1; i < kNoAllocSlots; ++i)
            if (d.last_use[i] < d.last_use[pick]) pick = i;
        e = hipDeviceSynchronize();
        if (e != hipSuccess)
            return fail(ALJABR_ROCM_ERR_DEVICE, "attention_gqa_noalloc: draining the device for a slot: %s",
                        hipGetErrorString(e));
    }
    d.owner[pick] = s;
    d.taken[pick] = true;
    d.last_use[pick] = ++d.clock;
    *out = d.base + static_cast<size_t>(pick) * (kNoAllocSlotBytes / sizeof(float));
    return ALJABR_ROCM_OK;
}

}  // namespace

extern "C" int aljabr_rocm_attention_gqa_noalloc(void *out, const void *Q, const void *K, const void *V,
                                                 const void *mask, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                                                 int kvType, float scale, int causal) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(out && Q && K && V, "out, Q, K and V must be non-null device pointers");
    ALJ_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Sq > 0 && Sk > 0 && D > 0 && Hq % Hkv == 0,
                "GQA expects Q[B,Hq,Sq,D], K/V[B,Hkv,Sk,D] with Hq divisible by Hkv");
    if (kvType != ALJABR_ROCM_TYPE_F32 && kvType != ALJABR_ROCM_TYPE_F16)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "attention: K/V type %d is not F32 or F16", kvType);
    if (mask)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED,
                    "attention_gqa_noalloc takes no mask (its check copies a flag to the host); use "
                    "aljabr_rocm_attention_gqa");
    // Two splits of partials for every query row must fit a slot, so that
    // the split count can always be lowered to what it holds.
    const size_t rows = static_cast<size_t>(B) * Hq * Sq;
    if (rows * 2 * (static_cast<size_t>(D) + 2) * sizeof(float) > kNoAllocSlotBytes)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT,
                    "attention_gqa_noalloc: B*Hq*Sq*2*(D+2)*4 = %zu bytes exceeds its %zu-byte scratch slot",
                    rows * 2 * (static_cast<size_t>(D) + 2) * sizeof(float), kNoAllocSlotBytes);
    AttnParams p{};
    p.out = static_cast<float *>(out);
    p.q = static_cast<const float *>(Q);
    p.k = K;
    p.v = V;
    p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Sq = Sq; p.Sk = Sk; p.D = D; p.cap = Sk;
    p.scale = scale > 0.0f ? scale : static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
    p.causal = causal != 0;
    p.kv_f16 = kvType == ALJABR_ROCM_TYPE_F16;
    p.scratch_bytes = kNoAllocSlotBytes;
    p.scratch_only = 1;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        float *buf = nullptr;
        int rc = noalloc_slot(current_stream(), &buf);
        if (rc) return rc;
        p.scratch = buf;
        rc = enqueue_attention(p);
        if (rc) return rc;
    }
    return finish_launch("attention_gqa_noalloc");
}

namespace aljabr {
namespace {

// Paged-table validation of aljabr_metal_attention_impl's CPU path
// (MTLC/aljabr_metal_attention.m:203-226): a sequence may not need more than
// max_blocks blocks, and every block it uses must be a non-negative index.
__global__ void paged_check_kernel(const int *__restrict__ block_table, const int *__restrict__ context_lens, int B,
                                   int block_size, int max_blocks, int *__restrict__ bad) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long long>(B) * max_blocks) return;
    const int b = static_cast<int>(i / max_blocks), blk = static_cast<int>(i % max_blocks);
    const int ctx = context_lens[b];
    if (ctx <= 0) return;
    const long long need = (static_cast<long long>(ctx) + block_size - 1) / block_size;
    if (blk == 0 && need > max_blocks) atomicOr(bad, 1);
    if (blk < need && block_table[i] < 0) atomicOr(bad, 1);
}

int paged_attention(void *out, const void *Q, const void *K_cache, const void *V_cache, const int *block_table,
                    const int *context_lens, int B, int T, int H, int H_kv, int D, int block_size, int max_blocks,
                    float scale, int is_causal, int query_start_pos, int sliding_window, float soft_cap) {
    ALJ_CHECK_READY();
    // Status codes as aljabr_metal_attention_impl (MTLC/aljabr_metal_attention.m:166-172).
    if (H_kv <= 0 || H % H_kv != 0)
        return fail(ALJABR_ROCM_ERR_NOT_INITIALIZED, "paged attention: H=%d is not a multiple of H_kv=%d", H, H_kv);
    if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || block_size <= 0 || max_blocks <= 0)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "paged attention: dimensions must be positive");
    ALJ_REQUIRE(out && Q && K_cache && V_cache && block_table && context_lens,
                "out, Q, K_cache, V_cache, block_table and context_lens must be non-null device pointers");
    ALJ_REQUIRE(static_cast<long long>(max_blocks) * block_size < (1LL << 31), "max_blocks * block_size too large");
    hipStream_t s = current_stream();
    int *flag = static_cast<int *>(stream_scratch(sizeof(int)));
    if (!flag) return ALJABR_ROCM_ERR_BUFFER;
    const long long n = static_cast<long long>(B) * max_blocks;
    hipLaunchKernelGGL(zero_i32_kernel, dim3(1), dim3(1), 0, s, flag);
    hipLaunchKernelGGL(paged_check_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, block_table,
                       context_lens, B, block_size, max_blocks, flag);
    int bad = 0;
    hipError_t e = hipMemcpyAsync(&bad, flag, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "paged attention table check: %s", hipGetErrorString(e));
    if (bad)
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT,
                    "paged attention: a context needs more than max_blocks blocks or a block index is negative");
    AttnParams p{};
    p.out = static_cast<float *>(out);
    p.q = static_cast<const float *>(Q);
    p.k = K_cache;
    p.v = V_cache;
    p.kv_len = context_lens;
    p.B = B; p.Hq = H; p.Hkv = H_kv; p.Sq = T; p.D = D;
    p.Sk = max_blocks * block_size;
    p.cap = 0;
    p.scale = scale;
    p.causal = is_causal != 0;
    p.kv_f16 = 0;
    p.block_table = block_table;
    p.block_size = block_size;
    p.max_blocks = max_blocks;
    p.paged_bounds = 1;
    p.query_start = query_start_pos;
    p.window = sliding_window;
    p.soft_cap = soft_cap;
    p.norm_eps = 1e-9f;                          // inv_sum = 1 / (sum + 1e-9)
    // Q and out are [B][T][H][D].
    p.q_sq = static_cast<long long>(H) * D;
    p.q_sh = D;
    p.q_sb = static_cast<long long>(T) * H * D;
    const int rc = enqueue_attention(p);
    if (rc) return rc;
    return finish_launch("paged_attention");
}

}  // namespace
}  // namespace aljabr

extern "C" {

int aljabr_rocm_paged_attention(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                const int *block_table, const int *context_lens, int B, int T, int H, int D,
                                int block_size, int max_blocks, float scale, int is_causal, float soft_cap) {
    return paged_attention(out, Q, K_cache, V_cache, block_table, context_lens, B, T, H, H, D, block_size, max_blocks,
                           scale, is_causal, 0, 0, soft_cap);
}

int aljabr_rocm_paged_attention_windowed(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                         const int *block_table, const int *context_lens, int B, int T, int H, int D,
                                         int block_size, int max_blocks, float scale, int is_causal,
                                         int query_start_pos, int sliding_window, float soft_cap) {
    return paged_attention(out, Q, K_cache, V_cache, block_table, context_lens, B, T, H, H, D, block_size, max_blocks,
                           scale, is_causal, query_start_pos, sliding_window, soft_cap);
}

int aljabr_rocm_paged_attention_gqa(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                    const int *block_table, const int *context_lens, int B, int T, int H, int H_kv,
                                    int D, int block_size, int max_blocks, float scale, int is_causal,
                                    float soft_cap) {
    return paged_attention(out, Q, K_cache, V_cache, block_table, context_lens, B, T, H, H_kv, D, block_size,
                           max_blocks, scale, is_causal, 0, 0, soft_cap);
}

int aljabr_rocm_paged_attention_gqa_windowed(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                             const int *block_table, const int *context_lens, int B, int T, int H,
                                             int H_kv, int D, int block_size, int max_blocks, float scale,
                                             int is_causal, int query_start_pos, int sliding_window, float soft_cap) {
    return paged_attention(out, Q, K_cache, V_cache, block_table, context_lens, B, T, H, H_kv, D, block_size,
                           max_blocks, scale, is_causal, query_start_pos, sliding_window, soft_cap);
}

}  // extern "C"
