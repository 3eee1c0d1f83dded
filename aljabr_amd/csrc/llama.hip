// llama.hip - device-resident Llama-style decode step over NF4 or GGUF-typed
// weights (F32, F16, Q4_0, Q8_0, Q4_K, Q6_K; any mix per matrix).
//
// Composition follows GgufDecodePass.forward's per-op path
// (engine/gguf/aljabr-gguf-java/src/main/java/tech/kayys/aljabr/gguf/javabackend/
// GgufDecodePass.java:297-505) and GgufLogitsProcessor.compute (:26-48):
//   x = embed[token]
//   per layer: xb = rmsNorm(x); q,k,v = Wq/Wk/Wv xb; rope(q,k); append k,v;
//              att = GQA(q, Kcache, Vcache); x += Wo att;
//              xb = rmsNorm(x); x += Wdown (silu(Wgate xb) * Wup xb)
//   logits = LMhead rmsNorm(x); next = argmax(logits)
// Unlike the reference's host-side loop, the whole step is enqueued on one
// stream with no host round trip; sequences of a batch are decoded together,
// so every weight byte is read once per step for the whole batch. The KV
// cache is fp16 [layer][batch][kv_head][max_seq][head_dim].
#include <algorithm>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "device.hpp"
#include "gguf.hpp"
#include "internal.hpp"
#include "safetensors.hpp"
#include "kernels.hpp"

namespace aljabr {

namespace {

__global__ void lengths_from_positions(int *__restrict__ len, const int *__restrict__ pos, int n) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) len[i] = pos[i] + 1;
}

// dst_a[i] = src_a[i], dst_b[i] = src_b[i] for i < n (either pair may be null).
__global__ void copy_i32_pairs(int *__restrict__ dst_a, const int *__restrict__ src_a, int *__restrict__ dst_b,
                               const int *__restrict__ src_b, int n) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) {
        if (dst_a) dst_a[i] = src_a[i];
        if (dst_b) dst_b[i] = src_b[i];
    }
}

}  // namespace
}  // namespace aljabr

struct aljabr_rocm_llama {
    // A weight matrix: device data, its ALJABR_ROCM_TYPE_* and (NF4) absmax.
    struct T {
        const uint8_t *w = nullptr;
        const float *s = nullptr;
        int type = ALJABR_ROCM_TYPE_NF4;
    };
    aljabr_rocm_llama_config cfg;
    std::vector<const float *> attn_norm, ffn_norm;
    std::vector<T> wq, wk, wv, wo, w_gate, w_up, w_down;
    T tok_embed, lm_head;
    const float *out_norm = nullptr;
    bool all_nf4 = true;      // every projection NF4 with cfg.nf4_block: the fused NF4 launches apply
    void *weights_owned = nullptr;   // device weights the session allocated (GGUF loader), freed with it
    void *arena = nullptr;   // one allocation for the KV cache and activations
    uint16_t *k_cache = nullptr, *v_cache = nullptr;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float *gate = nullptr, *up = nullptr, *hb = nullptr, *logits = nullptr;
    int *kv_len = nullptr;
    int *tok_in = nullptr, *pos_in = nullptr, *next_out = nullptr;   // graph replays read and write these
    float2 *rope_cs = nullptr;   // [max_seq][head_dim/2] RoPE cos/sin, filled at creation
    float *attn_scratch = nullptr;   // split-attention partials (owned: a captured graph keeps the address)
    size_t attn_scratch_bytes = 0;
    float *mm_part = nullptr;        // K-slice partials of the batched matrix-core GEMMs
    size_t mm_part_floats = 0;
    float *tail_ssq = nullptr;       // [max_batch][kSsqParts] row-block sums of squares of the residual tails
    // xb and hb as the NF4 GEMM's fp16 A image, written by the tails that
    // produce them (batches of 2..64): the next GEMM then skips its packing
    // launch. Null when the session has none.
    uint16_t *xb_pack = nullptr, *hb_pack = nullptr;
    uint16_t *att_pack = nullptr;    // the attention output's A image, written by the attention kernels
    bool rows_fused = false;   // batch-1 layers as fused NF4 launches (shapes and alignment allow it)
    // Captured decode steps, by batch size (and the logits buffer they write).
    struct Graph {
        hipGraphExec_t exec = nullptr;
        float *logits = nullptr;
    };
    std::vector<Graph> graphs;
};

using namespace aljabr;

namespace {

template <class T>
T *carve(char *&cursor, size_t count) {
    T *p = reinterpret_cast<T *>(cursor);
    cursor += (count * sizeof(T) + 255) & ~static_cast<size_t>(255);
    return p;
}

bool matvec_type(int t) {
    return t == ALJABR_ROCM_TYPE_NF4 || t == ALJABR_ROCM_TYPE_F32 || t == ALJABR_ROCM_TYPE_F16 ||
           t == ALJABR_ROCM_TYPE_Q4_0 || t == ALJABR_ROCM_TYPE_Q8_0 || t == ALJABR_ROCM_TYPE_Q4_K ||
           t == ALJABR_ROCM_TYPE_Q6_K;
}

// Elements per quantization block of a GGUF type (the row length must be a
// multiple), 1 for F32/F16.
int type_block(int t) {
    switch (t) {
    case ALJABR_ROCM_TYPE_Q4_0:
    case ALJABR_ROCM_TYPE_Q8_0: return 32;
    case ALJABR_ROCM_TYPE_Q4_K:
    case ALJABR_ROCM_TYPE_Q6_K: return 256;
    default: return 1;
    }
}

// Copies one typed matrix; rows of `k` elements must be whole blocks.
bool take_tensor(aljabr_rocm_llama::T &dst, const aljabr_rocm_tensor &src, int k, int nf4_block) {
    if (!src.data || !matvec_type(src.type) || k % type_block(src.type) != 0) return false;
    if (src.type == ALJABR_ROCM_TYPE_NF4 && (!src.absmax || (src.block_size != 0 && src.block_size != nf4_block)))
        return false;
    dst.w = static_cast<const uint8_t *>(src.data);
    dst.s = static_cast<const float *>(src.absmax);
    dst.type = src.type;
    return true;
}

int validate_config(const aljabr_rocm_llama_config &c) {
    ALJ_REQUIRE(c.layers > 0 && c.dim > 0 && c.ffn > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.head_dim > 0 &&
                    c.vocab > 0 && c.max_seq > 0 && c.max_batch > 0 && c.nf4_block > 0,
                "llama config dimensions must be positive");
    ALJ_REQUIRE(c.n_heads % c.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    ALJ_REQUIRE(c.head_dim % 2 == 0 && c.nf4_block % 2 == 0, "head_dim and nf4_block must be even");
    ALJ_REQUIRE(c.rope_base > 1.0f && c.eps >= 0.0f, "rope_base must exceed 1 and eps be non-negative");
    return ALJABR_ROCM_OK;
}

int create_session(const aljabr_rocm_llama_config &c, const aljabr_rocm_llama_tensors *w, aljabr_rocm_llama **out);

}  // namespace

extern "C" {

int aljabr_rocm_llama_create(const aljabr_rocm_llama_config *cfg, const aljabr_rocm_llama_weights *w,
                             aljabr_rocm_llama **out) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(cfg && w && out, "cfg, weights and out must be non-null");
    *out = nullptr;
    int rc = validate_config(*cfg);
    if (rc != ALJABR_ROCM_OK) return rc;
    ALJ_REQUIRE(w->tok_embed && w->out_norm && w->lm_head, "embedding, output norm and LM head are required");
    const int L = cfg->layers;
    ALJ_REQUIRE(w->attn_norm && w->ffn_norm && w->wq && w->wk && w->wv && w->wo && w->w_gate && w->w_up && w->w_down &&
                    w->wq_absmax && w->wk_absmax && w->wv_absmax && w->wo_absmax && w->w_gate_absmax &&
                    w->w_up_absmax && w->w_down_absmax,
                "every per-layer weight table must be non-null");
    // The NF4 layout as typed tensors (fp32 embedding, fp16 LM head).
    std::vector<aljabr_rocm_tensor> t(static_cast<size_t>(7) * L);
    auto nf4 = [&](const void *data, const void *absmax) {
        return aljabr_rocm_tensor{data, absmax, ALJABR_ROCM_TYPE_NF4, cfg->nf4_block};
    };
    for (int l = 0; l < L; ++l) {
        t[0 * L + l] = nf4(w->wq[l], w->wq_absmax[l]);
        t[1 * L + l] = nf4(w->wk[l], w->wk_absmax[l]);
        t[2 * L + l] = nf4(w->wv[l], w->wv_absmax[l]);
        t[3 * L + l] = nf4(w->wo[l], w->wo_absmax[l]);
        t[4 * L + l] = nf4(w->w_gate[l], w->w_gate_absmax[l]);
        t[5 * L + l] = nf4(w->w_up[l], w->w_up_absmax[l]);
        t[6 * L + l] = nf4(w->w_down[l], w->w_down_absmax[l]);
    }
    aljabr_rocm_llama_tensors tw{};
    tw.tok_embed = aljabr_rocm_tensor{w->tok_embed, nullptr, ALJABR_ROCM_TYPE_F32, 0};
    tw.attn_norm = w->attn_norm;
    tw.ffn_norm = w->ffn_norm;
    tw.wq = &t[0 * L];
    tw.wk = &t[1 * L];
    tw.wv = &t[2 * L];
    tw.wo = &t[3 * L];
    tw.w_gate = &t[4 * L];
    tw.w_up = &t[5 * L];
    tw.w_down = &t[6 * L];
    tw.out_norm = w->out_norm;
    tw.lm_head = aljabr_rocm_tensor{w->lm_head, nullptr, ALJABR_ROCM_TYPE_F16, 0};
    return create_session(*cfg, &tw, out);
}

int aljabr_rocm_llama_create_typed(const aljabr_rocm_llama_config *cfg, const aljabr_rocm_llama_tensors *w,
                                   aljabr_rocm_llama **out) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(cfg && w && out, "cfg, weights and out must be non-null");
    *out = nullptr;
    const int rc = validate_config(*cfg);
    if (rc != ALJABR_ROCM_OK) return rc;
    return create_session(*cfg, w, out);
}

}  // extern "C"

namespace {

int create_session(const aljabr_rocm_llama_config &c, const aljabr_rocm_llama_tensors *w, aljabr_rocm_llama **out) {
    ALJ_REQUIRE(w->out_norm && w->attn_norm && w->ffn_norm && w->wq && w->wk && w->wv && w->wo && w->w_gate &&
                    w->w_up && w->w_down,
                "output norm and every per-layer table are required");
    aljabr_rocm_llama *m = new (std::nothrow) aljabr_rocm_llama();
    if (!m) return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    m->cfg = c;
    const int L = c.layers;
    const int qd_i = c.n_heads * c.head_dim, kvd_i = c.n_kv_heads * c.head_dim;
    bool ok = true;
    m->attn_norm.resize(L);
    m->ffn_norm.resize(L);
    for (auto *v : {&m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up, &m->w_down}) v->resize(L);
    for (int l = 0; l < L && ok; ++l) {
        m->attn_norm[l] = static_cast<const float *>(w->attn_norm[l]);
        m->ffn_norm[l] = static_cast<const float *>(w->ffn_norm[l]);
        ok = m->attn_norm[l] && m->ffn_norm[l] && take_tensor(m->wq[l], w->wq[l], c.dim, c.nf4_block) &&
             take_tensor(m->wk[l], w->wk[l], c.dim, c.nf4_block) && take_tensor(m->wv[l], w->wv[l], c.dim, c.nf4_block) &&
             take_tensor(m->wo[l], w->wo[l], qd_i, c.nf4_block) &&
             take_tensor(m->w_gate[l], w->w_gate[l], c.dim, c.nf4_block) &&
             take_tensor(m->w_up[l], w->w_up[l], c.dim, c.nf4_block) &&
             take_tensor(m->w_down[l], w->w_down[l], c.ffn, c.nf4_block);
    }
    (void)kvd_i;
    const int et = w->tok_embed.type;
    ok = ok && w->tok_embed.data && et != ALJABR_ROCM_TYPE_NF4 && matvec_type(et) && c.dim % type_block(et) == 0 &&
         take_tensor(m->lm_head, w->lm_head, c.dim, c.nf4_block);
    if (!ok) {
        delete m;
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT,
                    "every weight must be non-null, of a supported type, with rows of whole blocks "
                    "(the embedding F32/F16/Q4_0/Q8_0/Q4_K/Q6_K; NF4 with absmax and the config's block size)");
    }
    m->tok_embed.w = static_cast<const uint8_t *>(w->tok_embed.data);
    m->tok_embed.type = et;
    m->out_norm = static_cast<const float *>(w->out_norm);
    for (int l = 0; l < L; ++l)
        for (const auto *v : {&m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up, &m->w_down})
            m->all_nf4 = m->all_nf4 && (*v)[l].type == ALJABR_ROCM_TYPE_NF4;

    const size_t B = static_cast<size_t>(c.max_batch);
    const size_t kvd = static_cast<size_t>(c.n_kv_heads) * c.head_dim;
    const size_t qd = static_cast<size_t>(c.n_heads) * c.head_dim;
    const size_t cache_elems = static_cast<size_t>(L) * B * kvd * c.max_seq;
    // K-slice partials of every matrix-core GEMM a step of 2..max_batch
    // tokens launches (stacked Q/K/V and gate/up, each projection alone, the
    // output head), so that no launch takes the stream's scratch: a captured
    // step keeps the addresses it was captured with.
    size_t mm_floats = 0;
    if (c.max_batch >= 2) {
        bool layer_nf4 = false, layer_kq = false;
        for (int l = 0; l < L; ++l)
            for (const auto *v : {&m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up, &m->w_down}) {
                layer_nf4 = layer_nf4 || (*v)[l].type == ALJABR_ROCM_TYPE_NF4;
                layer_kq = layer_kq || kquant_mfma_type((*v)[l].type);
            }
        const int ki = static_cast<int>(kvd), qi = static_cast<int>(qd);
        const int shapes[8][2] = {{qi + 2 * ki, c.dim}, {qi, c.dim}, {ki, c.dim}, {c.dim, qi},
                                  {2 * c.ffn, c.dim}, {c.ffn, c.dim}, {c.dim, c.ffn}, {c.vocab, c.dim}};
        for (int i = 0; i < 8; ++i) {
            const bool head = i == 7;
            const bool nf4 = head ? m->lm_head.type == ALJABR_ROCM_TYPE_NF4 : layer_nf4;
            const bool kq = head ? kquant_mfma_type(m->lm_head.type) : layer_kq;
            if (kq)
                mm_floats = std::max(mm_floats, kquant_mfma_scratch_floats(std::min(c.max_batch, 32), shapes[i][0],
                                                                           shapes[i][1]));
            for (int b = 2; nf4 && b <= c.max_batch; ++b)
                mm_floats = std::max(mm_floats, nf4_mfma_scratch_floats(b, shapes[i][0], shapes[i][1]));
        }
    }
    // The A images of xb, hb and the attention output for the NF4 GEMMs
    // (batches of 2..64), and of xb for Q4_K gate/up projections on the
    // register-resident kernel (K = dim a multiple of 4096).
    bool q4k_ffn = c.dim % 4096 == 0;
    for (int l = 0; l < L; ++l)
        q4k_ffn = q4k_ffn && m->w_gate[l].type == ALJABR_ROCM_TYPE_Q4_K && m->w_up[l].type == ALJABR_ROCM_TYPE_Q4_K;
    const bool packs = (m->all_nf4 || q4k_ffn) && c.max_batch >= 2 && c.max_batch <= 64 && c.dim % 64 == 0 &&
                       c.ffn % 64 == 0;
    const bool att_packs = m->all_nf4 && packs && qd % 64 == 0;
    const size_t pack_bytes = (packs ? ((nf4_xpack_bytes(c.max_batch, c.dim) + 255) & ~size_t(255)) +
                                           ((nf4_xpack_bytes(c.max_batch, c.ffn) + 255) & ~size_t(255))
                                     : 0) +
                              (att_packs ? (nf4_xpack_bytes(c.max_batch, static_cast<int>(qd)) + 255) & ~size_t(255) : 0);
    const size_t bytes = 2 * ((cache_elems * 2 + 255) & ~size_t(255)) +
                         ((mm_floats * 4 + 255) & ~size_t(255)) +
                         ((B * c.dim * 4 + 255) & ~size_t(255)) * 2 + ((B * qd * 4 + 255) & ~size_t(255)) * 2 +
                         ((B * kvd * 4 + 255) & ~size_t(255)) * 2 + ((B * c.ffn * 4 + 255) & ~size_t(255)) * 3 +
                         ((B * c.vocab * 4 + 255) & ~size_t(255)) + ((B * 4 + 255) & ~size_t(255)) * 4 +
                         ((attention_scratch_bytes(c.max_batch, c.n_heads, 1, c.head_dim, c.max_seq) + 255) &
                          ~size_t(255)) +
                         ((static_cast<size_t>(c.max_seq) * (c.head_dim / 2) * sizeof(float2) + 255) & ~size_t(255)) +
                         ((static_cast<size_t>(B) * kSsqParts * 4 + 255) & ~size_t(255)) + 256 + pack_bytes;
    hipError_t e = hipMalloc(&m->arena, bytes);
    if (e != hipSuccess) {
        delete m;
        return fail(ALJABR_ROCM_ERR_BUFFER, "llama session: hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    char *cur = static_cast<char *>(m->arena);
    m->k_cache = carve<uint16_t>(cur, cache_elems);
    m->v_cache = carve<uint16_t>(cur, cache_elems);
    m->x = carve<float>(cur, B * c.dim);
    m->xb = carve<float>(cur, B * c.dim);
    m->q = carve<float>(cur, B * qd);
    m->att = carve<float>(cur, B * qd);
    m->k = carve<float>(cur, B * kvd);
    m->v = carve<float>(cur, B * kvd);
    m->gate = carve<float>(cur, B * c.ffn);
    m->up = carve<float>(cur, B * c.ffn);
    m->hb = carve<float>(cur, B * c.ffn);
    m->logits = carve<float>(cur, B * c.vocab);
    m->kv_len = carve<int>(cur, B);
    m->tok_in = carve<int>(cur, B);
    m->pos_in = carve<int>(cur, B);
    m->next_out = carve<int>(cur, B);
    m->attn_scratch_bytes = attention_scratch_bytes(c.max_batch, c.n_heads, 1, c.head_dim, c.max_seq);
    m->attn_scratch = carve<float>(cur, m->attn_scratch_bytes / sizeof(float));
    if (c.max_batch >= 2) {
        m->mm_part_floats = mm_floats;
        m->mm_part = carve<float>(cur, mm_floats);
    }
    m->tail_ssq = carve<float>(cur, static_cast<size_t>(B) * kSsqParts);
    if (packs) {
        m->xb_pack = carve<uint16_t>(cur, nf4_xpack_bytes(c.max_batch, c.dim) / 2);
        m->hb_pack = carve<uint16_t>(cur, nf4_xpack_bytes(c.max_batch, c.ffn) / 2);
    }
    if (att_packs) m->att_pack = carve<uint16_t>(cur, nf4_xpack_bytes(c.max_batch, static_cast<int>(qd)) / 2);
    // The RoPE angles of every cache position, computed once: the decode
    // step then reads cos/sin instead of evaluating double pow/cos/sin.
    m->rope_cs = carve<float2>(cur, static_cast<size_t>(c.max_seq) * (c.head_dim / 2));
    int trc = enqueue_rope_table(m->rope_cs, c.max_seq, c.head_dim, c.rope_base);
    if (trc == ALJABR_ROCM_OK) trc = finish_launch("llama session: RoPE table");
    if (trc == ALJABR_ROCM_OK) {
        const hipError_t se = hipStreamSynchronize(current_stream());
        if (se != hipSuccess) trc = fail(ALJABR_ROCM_ERR_DEVICE, "llama session: RoPE table: %s", hipGetErrorString(se));
    }
    if (trc != ALJABR_ROCM_OK) {
        (void)hipFree(m->arena);
        delete m;
        return trc;
    }
    m->graphs.resize(static_cast<size_t>(c.max_batch) + 1);
    // Batch-1 fusion (the rows kernels: NF4, Q4_0, Q8_0, Q4_K, Q6_K) needs
    // every K a multiple of 2048 (at most 16384), for NF4 a power-of-two block
    // of at least 32, and 16-byte aligned weights and norms.
    const int shift = log2_exact(c.nf4_block);
    auto k_ok = [](int k) { return k % 2048 == 0 && k / 2048 >= 1 && k / 2048 <= 8; };
    auto rows_type = [&](int t) {
        return (t == ALJABR_ROCM_TYPE_NF4 && shift >= 5) || t == ALJABR_ROCM_TYPE_Q4_0 || t == ALJABR_ROCM_TYPE_Q8_0 ||
               t == ALJABR_ROCM_TYPE_Q4_K || t == ALJABR_ROCM_TYPE_Q6_K;
    };
    bool fused = k_ok(c.dim) && k_ok(qd_i) && k_ok(c.ffn);
    for (int l = 0; l < L && fused; ++l)
        for (const auto *t : {&m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up, &m->w_down})
            fused = fused && rows_type((*t)[l].type);
    for (int l = 0; l < L && fused; ++l) {
        fused = aligned(m->attn_norm[l], 16) && aligned(m->ffn_norm[l], 16);
        for (const auto *t : {&m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up, &m->w_down})
            fused = fused && aligned((*t)[l].w, 16);
    }
    m->rows_fused = fused;
    *out = m;
    return ALJABR_ROCM_OK;
}

}  // namespace

namespace {

// binary16 bits -> binary32 (exact; NaN -> canonical quiet NaN).
float half_to_float(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int lz = 0;
            uint32_t mm = mant;
            while (!(mm & 0x400u)) {
                mm <<= 1;
                ++lz;
            }
            bits = (sign << 31) | ((113u - static_cast<uint32_t>(lz)) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = mant == 0 ? ((sign << 31) | 0x7f800000u) : 0x7fc00000u;
    } else {
        bits = (sign << 31) | ((e + 112u) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Metadata lookups of a Llama-family GGUF file ("{arch}.key").
struct GgufMeta {
    const GgufFile &g;
    std::string arch;
    bool num(const std::string &key, double &v) const {
        const GgufValue *x = g.find(arch + "." + key);
        if (!x || x->type == 8 || x->type == 9) return false;
        v = (x->type == 6 || x->type == 12) ? x->f : static_cast<double>(x->i);
        return true;
    }
};

}  // namespace

extern "C" {

int aljabr_rocm_llama_create_gguf(const char *path, int max_batch, int max_seq, aljabr_rocm_llama **out) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(path && out && max_batch > 0, "path, out and a positive max_batch are required");
    *out = nullptr;
    GgufFile *raw = nullptr;
    int rc = gguf_open(path, &raw);
    if (rc != ALJABR_ROCM_OK) return rc;
    std::unique_ptr<GgufFile> g(raw);
    GgufMeta meta{*g, "llama"};
    if (const GgufValue *a = g->find("general.architecture"))
        if (a->type == 8) meta.arch = a->s;
    double v;
    aljabr_rocm_llama_config c{};
    auto need = [&](const char *key, int32_t &dst) {
        if (!meta.num(key, v)) return false;
        dst = static_cast<int32_t>(v);
        return true;
    };
    if (!need("block_count", c.layers) || !need("embedding_length", c.dim) || !need("feed_forward_length", c.ffn) ||
        !need("attention.head_count", c.n_heads))
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: %s lacks %s.block_count / embedding_length / "
                    "feed_forward_length / attention.head_count", path, meta.arch.c_str());
    c.n_kv_heads = meta.num("attention.head_count_kv", v) ? static_cast<int32_t>(v) : c.n_heads;
    c.head_dim = meta.num("attention.key_length", v) ? static_cast<int32_t>(v)
                                                       : (c.n_heads > 0 ? c.dim / c.n_heads : 0);
    c.rope_base = meta.num("rope.freq_base", v) ? static_cast<float>(v) : 10000.0f;
    c.eps = meta.num("attention.layer_norm_rms_epsilon", v) ? static_cast<float>(v) : 1e-5f;
    c.max_seq = max_seq > 0 ? max_seq : (meta.num("context_length", v) ? static_cast<int32_t>(v) : 0);
    c.max_batch = max_batch;
    c.nf4_block = 64;
    if (meta.num("rope.dimension_count", v) && static_cast<int32_t>(v) != c.head_dim)
        return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "gguf: %s rotates %d of %d head dimensions (partial RoPE)", path,
                    static_cast<int>(v), c.head_dim);
    // Tensors the decode step does not apply: refuse rather than decode a
    // different model.
    for (const char *extra : {"blk.0.attn_q_norm.weight", "blk.0.attn_k_norm.weight", "blk.0.post_attention_norm.weight",
                              "blk.0.post_ffw_norm.weight", "rope_freqs.weight", "blk.0.rope_freqs.weight",
                              "blk.0.layer_output_scale.weight", "blk.0.attn_q.bias", "blk.0.attn_v_norm.weight"})
        if (g->tensor(extra))
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "gguf: %s has %s, which this decode step does not apply", path,
                        extra);
    const GgufTensor *emb = g->tensor("token_embd.weight");
    ALJ_REQUIRE(emb && emb->n_dims == 2 && emb->dims[0] == c.dim, "gguf: %s: token_embd.weight must be [%d, vocab]",
                path, c.dim);
    c.vocab = static_cast<int32_t>(emb->dims[1]);
    rc = validate_config(c);
    if (rc != ALJABR_ROCM_OK) return rc;
    const int L = c.layers;
    const int64_t qd = static_cast<int64_t>(c.n_heads) * c.head_dim, kvd = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;

    // Every tensor the step reads, with its expected [K, N] shape (GGUF dims:
    // ne0 = row length K, ne1 = rows N).
    struct Need {
        const GgufTensor *t;
        int64_t k, n;
        bool norm;
    };
    std::vector<Need> needs;
    auto want = [&](const std::string &name, int64_t k, int64_t n, bool norm) -> int {
        const GgufTensor *t = g->tensor(name);
        if (!t) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: %s: missing tensor %s", path, name.c_str());
        const bool shape = norm ? (t->n_dims == 1 && t->dims[0] == k) : (t->n_dims == 2 && t->dims[0] == k && t->dims[1] == n);
        if (!shape) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "gguf: %s: tensor %s has the wrong shape", path, name.c_str());
        const bool ok_type = norm ? (t->type == ALJABR_ROCM_TYPE_F32 || t->type == ALJABR_ROCM_TYPE_F16)
                                  : matvec_type(t->type) && t->type != ALJABR_ROCM_TYPE_NF4 && k % type_block(t->type) == 0;
        if (!ok_type)
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "gguf: %s: tensor %s has type %d (supported: F32, F16, Q4_0, "
                        "Q8_0, Q4_K, Q6_K)", path, name.c_str(), t->type);
        needs.push_back({t, k, n, norm});
        return ALJABR_ROCM_OK;
    };
    rc = want("token_embd.weight", c.dim, c.vocab, false);
    for (int l = 0; l < L && rc == ALJABR_ROCM_OK; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        rc = want(b + "attn_norm.weight", c.dim, 1, true);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "attn_q.weight", c.dim, qd, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "attn_k.weight", c.dim, kvd, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "attn_v.weight", c.dim, kvd, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "attn_output.weight", qd, c.dim, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "ffn_norm.weight", c.dim, 1, true);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "ffn_gate.weight", c.dim, c.ffn, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "ffn_up.weight", c.dim, c.ffn, false);
        if (rc == ALJABR_ROCM_OK) rc = want(b + "ffn_down.weight", c.ffn, c.dim, false);
    }
    if (rc == ALJABR_ROCM_OK) rc = want("output_norm.weight", c.dim, 1, true);
    const bool tied = g->tensor("output.weight") == nullptr;     // LM head tied to the embedding
    if (rc == ALJABR_ROCM_OK && !tied) rc = want("output.weight", c.dim, c.vocab, false);
    if (rc != ALJABR_ROCM_OK) return rc;

    // One device allocation for every tensor (norms as fp32), 256-byte aligned.
    auto dev_bytes = [](const Need &n) { return n.norm ? static_cast<uint64_t>(n.k) * 4 : n.t->bytes; };
    uint64_t total = 0;
    for (const Need &n : needs) total += (dev_bytes(n) + 255) & ~uint64_t(255);
    void *base = nullptr;
    hipError_t e = hipMalloc(&base, total);
    if (e != hipSuccess)
        return fail(ALJABR_ROCM_ERR_BUFFER, "gguf: hipMalloc(%llu) for the weights: %s",
                    static_cast<unsigned long long>(total), hipGetErrorString(e));
    std::vector<const void *> dev(needs.size());
    uint64_t off = 0;
    std::vector<float> tmp;
    for (size_t i = 0; i < needs.size() && e == hipSuccess; ++i) {
        const Need &n = needs[i];
        char *dst = static_cast<char *>(base) + off;
        dev[i] = dst;
        if (n.norm && n.t->type == ALJABR_ROCM_TYPE_F16) {
            tmp.resize(static_cast<size_t>(n.k));
            const uint16_t *h = reinterpret_cast<const uint16_t *>(g->data(*n.t));
            for (int64_t j = 0; j < n.k; ++j) {
                uint16_t bits;
                std::memcpy(&bits, h + j, 2);
                tmp[static_cast<size_t>(j)] = half_to_float(bits);
            }
            e = hipMemcpy(dst, tmp.data(), static_cast<size_t>(n.k) * 4, hipMemcpyHostToDevice);
        } else {
            e = hipMemcpy(dst, g->data(*n.t), static_cast<size_t>(dev_bytes(n)), hipMemcpyHostToDevice);
        }
        off += (dev_bytes(n) + 255) & ~uint64_t(255);
    }
    if (e != hipSuccess) {
        (void)hipFree(base);
        return fail(ALJABR_ROCM_ERR_DEVICE, "gguf: uploading weights: %s", hipGetErrorString(e));
    }

    // needs[] order: embedding, 9 per layer, output norm, [output].
    auto tensor = [&](size_t i) { return aljabr_rocm_tensor{dev[i], nullptr, needs[i].t->type, 0}; };
    std::vector<aljabr_rocm_tensor> t(static_cast<size_t>(7) * L);
    std::vector<const void *> an(L), fn(L);
    for (int l = 0; l < L; ++l) {
        const size_t b = 1 + 9 * static_cast<size_t>(l);
        an[l] = dev[b];
        t[0 * L + l] = tensor(b + 1);
        t[1 * L + l] = tensor(b + 2);
        t[2 * L + l] = tensor(b + 3);
        t[3 * L + l] = tensor(b + 4);
        fn[l] = dev[b + 5];
        t[4 * L + l] = tensor(b + 6);
        t[5 * L + l] = tensor(b + 7);
        t[6 * L + l] = tensor(b + 8);
    }
    const size_t on = 1 + 9 * static_cast<size_t>(L);
    aljabr_rocm_llama_tensors tw{};
    tw.tok_embed = tensor(0);
    tw.attn_norm = an.data();
    tw.ffn_norm = fn.data();
    tw.wq = &t[0 * L];
    tw.wk = &t[1 * L];
    tw.wv = &t[2 * L];
    tw.wo = &t[3 * L];
    tw.w_gate = &t[4 * L];
    tw.w_up = &t[5 * L];
    tw.w_down = &t[6 * L];
    tw.out_norm = dev[on];
    tw.lm_head = tied ? tensor(0) : tensor(on + 1);
    aljabr_rocm_llama *m = nullptr;
    rc = create_session(c, &tw, &m);
    if (rc != ALJABR_ROCM_OK) {
        (void)hipFree(base);
        return rc;
    }
    m->weights_owned = base;
    *out = m;
    return ALJABR_ROCM_OK;
}

// A Llama model from a safetensors file with Hugging Face tensor names and
// NF4 projections in the safetensor engine's convention (AccelWeightBridge.
// java:184-222: "<name>.qweight" U8 [out, in/2] + "<name>.scales" fp32, group
// 128), dense projections F32 / F16 / BF16 (BF16 widened to fp32 exactly),
// norms and the embedding dense, the LM head dense, NF4 or tied to the
// embedding. The architecture comes from `cfg` (a safetensors file carries
// none); nf4_block is 128. Q and K rows are used as stored: the decode step's
// RoPE rotates (i, i + head_dim/2) pairs, the Hugging Face layout.
int aljabr_rocm_llama_create_safetensors(const char *path, const aljabr_rocm_llama_config *cfg,
                                         aljabr_rocm_llama **out) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(path && cfg && out, "path, cfg and out must be non-null");
    *out = nullptr;
    StFile *raw = nullptr;
    int rc = st_open(path, &raw);
    if (rc != ALJABR_ROCM_OK) return rc;
    std::unique_ptr<StFile> f(raw);
    aljabr_rocm_llama_config c = *cfg;
    c.nf4_block = 128;
    rc = validate_config(c);
    if (rc != ALJABR_ROCM_OK) return rc;
    for (const char *extra : {"model.layers.0.self_attn.q_norm.weight", "model.layers.0.self_attn.k_norm.weight",
                              "model.layers.0.self_attn.q_proj.bias", "model.layers.0.self_attn.k_proj.bias",
                              "model.layers.0.self_attn.v_proj.bias", "model.layers.0.pre_feedforward_layernorm.weight",
                              "model.layers.0.post_feedforward_layernorm.weight"})
        if (f->find(extra))
            return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "safetensors: %s has %s, which this decode step does not apply",
                        path, extra);
    const int L = c.layers;
    const int64_t qd = static_cast<int64_t>(c.n_heads) * c.head_dim, kvd = static_cast<int64_t>(c.n_kv_heads) * c.head_dim;

    // Every tensor the step reads: dense (`w`), or NF4 codes + scales.
    struct Need {
        const StTensor *w, *scales;
        int64_t n, k;           // rows, row length (norms: n = 1)
        int type;               // device type: F32, F16 or NF4
        bool norm;
    };
    std::vector<Need> needs;
    auto dense_type = [](int dt) {
        return dt == kStF32 || dt == kStBF16 ? ALJABR_ROCM_TYPE_F32 : dt == kStF16 ? ALJABR_ROCM_TYPE_F16 : -1;
    };
    auto want_norm = [&](const std::string &name) -> int {
        const StTensor *t = f->find(name);
        if (!t) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: missing tensor %s", path, name.c_str());
        if (t->shape.size() != 1 || t->shape[0] != c.dim || dense_type(t->dtype) < 0)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: %s must be a [%d] F32/F16/BF16 vector", path,
                        name.c_str(), c.dim);
        needs.push_back({t, nullptr, 1, c.dim, ALJABR_ROCM_TYPE_F32, true});
        return ALJABR_ROCM_OK;
    };
    auto want_matrix = [&](const std::string &base, int64_t n, int64_t k, bool allow_nf4) -> int {
        const StTensor *q = f->find(base + ".qweight");
        if (q) {
            const StTensor *sc = f->find(base + ".scales");
            if (!allow_nf4)
                return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "safetensors: %s: %s is NF4, which the embedding rows cannot "
                            "read", path, base.c_str());
            if (!sc || q->dtype != kStU8 || q->shape.size() != 2 || q->shape[0] != n || 2 * q->shape[1] != k)
                return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: %s.qweight must be U8 [%lld, %lld] with "
                            "%s.scales", path, base.c_str(), static_cast<long long>(n), static_cast<long long>(k / 2),
                            base.c_str());
            if (sc->dtype != kStF32 || k % c.nf4_block != 0 ||
                static_cast<int64_t>((sc->end - sc->begin) / 4) != n * k / c.nf4_block)
                return fail(ALJABR_ROCM_ERR_UNSUPPORTED, "safetensors: %s: %s.scales must hold one F32 absmax per "
                            "%d weights", path, base.c_str(), c.nf4_block);
            needs.push_back({q, sc, n, k, ALJABR_ROCM_TYPE_NF4, false});
            return ALJABR_ROCM_OK;
        }
        const StTensor *t = f->find(base + ".weight");
        if (!t) return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: missing tensor %s.weight / .qweight", path,
                            base.c_str());
        if (t->shape.size() != 2 || t->shape[0] != n || t->shape[1] != k || dense_type(t->dtype) < 0)
            return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "safetensors: %s: %s.weight must be a [%lld, %lld] F32/F16/BF16 "
                        "matrix", path, base.c_str(), static_cast<long long>(n), static_cast<long long>(k));
        needs.push_back({t, nullptr, n, k, dense_type(t->dtype), false});
        return ALJABR_ROCM_OK;
    };
    rc = want_matrix("model.embed_tokens", c.vocab, c.dim, false);
    for (int l = 0; l < L && rc == ALJABR_ROCM_OK; ++l) {
        const std::string b = "model.layers." + std::to_string(l) + ".";
        rc = want_norm(b + "input_layernorm.weight");
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "self_attn.q_proj", qd, c.dim, true);
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "self_attn.k_proj", kvd, c.dim, true);
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "self_attn.v_proj", kvd, c.dim, true);
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "self_attn.o_proj", c.dim, qd, true);
        if (rc == ALJABR_ROCM_OK) rc = want_norm(b + "post_attention_layernorm.weight");
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "mlp.gate_proj", c.ffn, c.dim, true);
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "mlp.up_proj", c.ffn, c.dim, true);
        if (rc == ALJABR_ROCM_OK) rc = want_matrix(b + "mlp.down_proj", c.dim, c.ffn, true);
    }
    if (rc == ALJABR_ROCM_OK) rc = want_norm("model.norm.weight");
    const bool tied = !f->find("lm_head.weight") && !f->find("lm_head.qweight");
    if (rc == ALJABR_ROCM_OK && !tied) rc = want_matrix("lm_head", c.vocab, c.dim, true);
    if (rc != ALJABR_ROCM_OK) return rc;

    // One device allocation: dense tensors as F32 (BF16 widened) or F16,
    // NF4 codes then absmax; 256-byte aligned pieces.
    auto main_bytes = [](const Need &n) -> uint64_t {
        const uint64_t e = static_cast<uint64_t>(n.n) * n.k;
        return n.type == ALJABR_ROCM_TYPE_NF4 ? e / 2 : n.type == ALJABR_ROCM_TYPE_F16 ? 2 * e : 4 * e;
    };
    auto align = [](uint64_t v) { return (v + 255) & ~uint64_t(255); };
    uint64_t total = 0;
    for (const Need &n : needs) total += align(main_bytes(n)) + (n.scales ? align(n.scales->end - n.scales->begin) : 0);
    void *base = nullptr;
    hipError_t e = hipMalloc(&base, total);
    if (e != hipSuccess)
        return fail(ALJABR_ROCM_ERR_BUFFER, "safetensors: hipMalloc(%llu) for the weights: %s",
                    static_cast<unsigned long long>(total), hipGetErrorString(e));
    std::vector<const void *> dev(needs.size()), dev_s(needs.size(), nullptr);
    uint64_t off = 0;
    std::vector<float> tmp;
    for (size_t i = 0; i < needs.size() && e == hipSuccess; ++i) {
        const Need &n = needs[i];
        char *dst = static_cast<char *>(base) + off;
        dev[i] = dst;
        const uint8_t *src = f->data(*n.w);
        if (n.w->dtype == kStBF16 || (n.norm && n.w->dtype == kStF16)) {
            const size_t cnt = static_cast<size_t>(n.n * n.k);
            tmp.resize(cnt);
            for (size_t j = 0; j < cnt; ++j) {
                uint16_t bits;
                std::memcpy(&bits, src + 2 * j, 2);
                if (n.w->dtype == kStBF16) {
                    const uint32_t wide = static_cast<uint32_t>(bits) << 16;
                    std::memcpy(&tmp[j], &wide, 4);
                } else {
                    tmp[j] = half_to_float(bits);
                }
            }
            e = hipMemcpy(dst, tmp.data(), cnt * 4, hipMemcpyHostToDevice);
        } else {
            e = hipMemcpy(dst, src, static_cast<size_t>(main_bytes(n)), hipMemcpyHostToDevice);
        }
        off += align(main_bytes(n));
        if (n.scales && e == hipSuccess) {
            char *sd = static_cast<char *>(base) + off;
            dev_s[i] = sd;
            e = hipMemcpy(sd, f->data(*n.scales), n.scales->end - n.scales->begin, hipMemcpyHostToDevice);
            off += align(n.scales->end - n.scales->begin);
        }
    }
    if (e != hipSuccess) {
        (void)hipFree(base);
        return fail(ALJABR_ROCM_ERR_DEVICE, "safetensors: uploading weights: %s", hipGetErrorString(e));
    }

    // needs[] order: embedding, 9 per layer, final norm, [lm_head].
    auto tensor = [&](size_t i) {
        return aljabr_rocm_tensor{dev[i], dev_s[i], needs[i].type, needs[i].type == ALJABR_ROCM_TYPE_NF4 ? c.nf4_block : 0};
    };
    std::vector<aljabr_rocm_tensor> t(static_cast<size_t>(7) * L);
    std::vector<const void *> an(L), fn(L);
    for (int l = 0; l < L; ++l) {
        const size_t b = 1 + 9 * static_cast<size_t>(l);
        an[l] = dev[b];
        t[0 * L + l] = tensor(b + 1);
        t[1 * L + l] = tensor(b + 2);
        t[2 * L + l] = tensor(b + 3);
        t[3 * L + l] = tensor(b + 4);
        fn[l] = dev[b + 5];
        t[4 * L + l] = tensor(b + 6);
        t[5 * L + l] = tensor(b + 7);
        t[6 * L + l] = tensor(b + 8);
    }
    const size_t on = 1 + 9 * static_cast<size_t>(L);
    aljabr_rocm_llama_tensors tw{};
    tw.tok_embed = tensor(0);
    tw.attn_norm = an.data();
    tw.ffn_norm = fn.data();
    tw.wq = &t[0 * L];
    tw.wk = &t[1 * L];
    tw.wv = &t[2 * L];
    tw.wo = &t[3 * L];
    tw.w_gate = &t[4 * L];
    tw.w_up = &t[5 * L];
    tw.w_down = &t[6 * L];
    tw.out_norm = dev[on];
    tw.lm_head = tied ? tensor(0) : tensor(on + 1);
    aljabr_rocm_llama *m = nullptr;
    rc = create_session(c, &tw, &m);
    if (rc != ALJABR_ROCM_OK) {
        (void)hipFree(base);
        return rc;
    }
    m->weights_owned = base;
    *out = m;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_llama_config_get(const aljabr_rocm_llama *m, aljabr_rocm_llama_config *cfg) {
    ALJ_REQUIRE(m && cfg, "model and cfg must be non-null");
    *cfg = m->cfg;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_llama_destroy(aljabr_rocm_llama *m) {
    if (!m) return ALJABR_ROCM_OK;
    ALJ_CHECK_READY();
    for (auto &g : m->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (m->arena) (void)hipFree(m->arena);
    if (m->weights_owned) (void)hipFree(m->weights_owned);
    delete m;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_llama_hidden(aljabr_rocm_llama *m, void **hidden) {
    ALJ_REQUIRE(m && hidden, "model and hidden must be non-null");
    *hidden = m->x;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_llama_kv_cache(aljabr_rocm_llama *m, void **k_cache, void **v_cache) {
    ALJ_REQUIRE(m && k_cache && v_cache, "model and cache out-pointers must be non-null");
    *k_cache = m->k_cache;
    *v_cache = m->v_cache;
    return ALJABR_ROCM_OK;
}

}  // extern "C"

namespace {

// Optional per-launch-group timing of a step: an event after every group on
// the step's stream, and the algorithmic bytes the group moves.
struct StepProfiler {
    std::vector<hipEvent_t> events;   // events[0] opens the step
    std::vector<const char *> names;
    std::vector<double> bytes;
    size_t used = 0;
    hipStream_t stream = nullptr;

    int begin(hipStream_t s, size_t groups) {
        stream = s;
        while (events.size() < groups + 1) {
            hipEvent_t e;
            const hipError_t r = hipEventCreate(&e);
            if (r != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipEventCreate: %s", hipGetErrorString(r));
            events.push_back(e);
        }
        used = 0;
        names.clear();
        bytes.clear();
        return record();
    }
    int record() {
        if (used >= events.size()) return fail(ALJABR_ROCM_ERR_BUFFER, "decode profile: out of events");
        const hipError_t r = hipEventRecord(events[used++], stream);
        return r == hipSuccess ? ALJABR_ROCM_OK : fail(ALJABR_ROCM_ERR_DEVICE, "hipEventRecord: %s", hipGetErrorString(r));
    }
    int mark(const char *name, double b) {
        names.push_back(name);
        bytes.push_back(b);
        return record();
    }
    ~StepProfiler() {
        for (hipEvent_t e : events) (void)hipEventDestroy(e);
    }
};

// NF4 weight bytes of an [n, k] matrix: codes + fp32 absmax.
double nf4_w(long long n, long long k, int bs) { return static_cast<double>(n * k / 2 + n * k / bs * 4); }

// Weight bytes of an [n, k] matrix of any type.
double weight_bytes(int type, long long n, long long k, int bs) {
    const double e = static_cast<double>(n) * k;
    switch (type) {
    case ALJABR_ROCM_TYPE_NF4: return nf4_w(n, k, bs);
    case ALJABR_ROCM_TYPE_F32: return 4.0 * e;
    case ALJABR_ROCM_TYPE_F16: return 2.0 * e;
    case ALJABR_ROCM_TYPE_Q4_0: return e / 32 * 18;
    case ALJABR_ROCM_TYPE_Q8_0: return e / 32 * 34;
    case ALJABR_ROCM_TYPE_Q4_K: return e / 256 * 144;
    case ALJABR_ROCM_TYPE_Q6_K: return e / 256 * 210;
    default: return 0.0;
    }
}

int decode_step(aljabr_rocm_llama *m, const int *tok, const int *pos, int B, float *lg, int *next,
                StepProfiler *prof, const int *host_pos) {
    const aljabr_rocm_llama_config &c = m->cfg;
    const int dim = c.dim, hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv_heads;
    const int qd = nh * hd, kvd = nkv * hd, ffn = c.ffn, bs = c.nf4_block;
    const int shift = log2_exact(bs);
    const size_t layer_cache = static_cast<size_t>(c.max_batch) * kvd * c.max_seq;
    const double f4 = 4.0;
    int rc;
#define ALJ_TRY(expr)                           \
    do {                                        \
        rc = (expr);                            \
        if (rc != ALJABR_ROCM_OK) return rc;    \
    } while (0)
#define ALJ_MARK(name, b)                                   \
    do {                                                    \
        if (prof) ALJ_TRY(prof->mark((name), (b)));         \
    } while (0)
    hipStream_t s = current_stream();
    // Visible keys summed over the batch (profiling only: bytes of the KV rows read).
    double keys = 0.0;
    if (host_pos)
        for (int b = 0; b < B; ++b) keys += std::min(host_pos[b] + 1, c.max_seq);
    using T = aljabr_rocm_llama::T;
    // y = x . W^T or, with `residual`, y += x . W^T for B rows. NF4 and the
    // GGUF block formats on the matrix cores add into y themselves when it
    // holds the residual; otherwise y is written, or the products go to `tmp`
    // and one add follows.
    auto mm = [&](float *y, const float *x, const T &t, int K, int N, bool residual, float *tmp) -> int {
        if (t.type == ALJABR_ROCM_TYPE_NF4 && B >= 2 && shift >= 0 && m->all_nf4) {
            const int r = enqueue_nf4_mfma(y, x, t.w, t.s, K, N, shift, B, residual, m->mm_part,
                                           m->mm_part_floats);
            if (r != ALJABR_ROCM_ERR_UNSUPPORTED) return r;
        }
        if (kquant_mfma_type(t.type) && B >= 2 && B <= kquant_mfma_max_m(t.type)) {
            const KqOut o{y, t.w, N};
            const int r = enqueue_kquant_mfma_multi(&o, 1, x, K, t.type, B, true, m->mm_part, m->mm_part_floats);
            if (r != ALJABR_ROCM_ERR_UNSUPPORTED) return r;
        }
        if (!residual) return enqueue_matmul_typed(y, x, t.w, t.s, t.type, bs, K, N, B, m->mm_part, m->mm_part_floats);
        const int r = enqueue_matmul_typed(tmp, x, t.w, t.s, t.type, bs, K, N, B, m->mm_part, m->mm_part_floats);
        if (r != ALJABR_ROCM_OK) return r;
        return enqueue_add(y, tmp, static_cast<long long>(B) * N);
    };
    // Matrices of one layer block: runs of one type go to the matrix cores as
    // one stacked launch where they can, the rest one by one.
    auto mm_run = [&](float *const *ys, const T *const *ts, const int *ns, int cnt, const float *x, int K) -> int {
        for (int i = 0; i < cnt;) {
            int j = i + 1;
            while (j < cnt && ts[j]->type == ts[i]->type) ++j;
            int r = ALJABR_ROCM_ERR_UNSUPPORTED;
            if (kquant_mfma_type(ts[i]->type) && B >= 2 && B <= kquant_mfma_max_m(ts[i]->type)) {
                KqOut o[3];
                for (int k = i; k < j; ++k) o[k - i] = KqOut{ys[k], ts[k]->w, ns[k]};
                r = enqueue_kquant_mfma_multi(o, j - i, x, K, ts[i]->type, B, false, m->mm_part, m->mm_part_floats);
            }
            if (r == ALJABR_ROCM_ERR_UNSUPPORTED) {
                for (int k = i; k < j; ++k) {
                    r = mm(ys[k], x, *ts[k], K, ns[k], false, nullptr);
                    if (r != ALJABR_ROCM_OK) return r;
                }
            } else if (r != ALJABR_ROCM_OK) {
                return r;
            }
            i = j;
        }
        return ALJABR_ROCM_OK;
    };
    // Bytes of one B-row product: weights once, activations in, outputs out
    // (read too when added into).
    auto mm_bytes = [&](const T &t, long long N, long long K, bool add) {
        return weight_bytes(t.type, N, K, bs) + B * (K + N * (add ? 2.0 : 1.0)) * f4;
    };
    const bool fused1 = B == 1 && m->rows_fused;
    // Batches of 2..32 over NF4 (block 64) or K-quant weights: each GEMM's
    // slice-sum kernel also runs the step that follows it (RoPE and the KV
    // append, the residual add and the next RMSNorm or its row-block sums,
    // SwiGLU). A GEMM the matrix cores do not take falls back to the separate
    // launches for that block only.
    const bool tails = !fused1 && B >= 2 && B <= 32 && (!m->all_nf4 || shift == 6);
    // One matrix-core GEMM over matrices of one type (NF4 or a K-quant) whose
    // slice sums go to the tail kernel `t`; UNSUPPORTED when the types or
    // shapes do not allow it (the caller then runs the separate launches).
    auto kq_ok = [&](const T &w) { return kquant_mfma_type(w.type) && B <= kquant_mfma_max_m(w.type); };
    auto gemm_tail = [&](const RowsOut *o, const T *const *ts, int nseg, const float *x, int K,
                         const SliceTail *t, const uint16_t *xpacked = nullptr) -> int {
        const int ty = ts[0]->type;
        bool mixed = false;
        for (int i = 1; i < nseg; ++i) mixed |= ts[i]->type != ty;
        if (mixed) {
            // K-quants of different types: one launch per run of one type,
            // each into its columns of one partial-sum buffer, then the tail.
            int n_all = 0;
            for (int i = 0; i < nseg; ++i) {
                if (!kq_ok(*ts[i])) return ALJABR_ROCM_ERR_UNSUPPORTED;
                n_all += o[i].n;
            }
            const int slices = K / 512;
            if (K % 512 != 0 || slices < 2 || static_cast<size_t>(slices) * B * n_all > m->mm_part_floats)
                return ALJABR_ROCM_ERR_UNSUPPORTED;
            // Two runs (Q4_K q and k, then a Q6_K v): one launch of both.
            int j0 = 1;
            while (j0 < nseg && ts[j0]->type == ty) ++j0;
            bool two_runs = j0 < nseg;
            for (int u = j0 + 1; u < nseg; ++u) two_runs &= ts[u]->type == ts[j0]->type;
            if (two_runs) {
                KqOut k0[3], k1[3];
                for (int u = 0; u < nseg; ++u)
                    (u < j0 ? k0[u] : k1[u - j0]) = KqOut{o[u].y, o[u].w, o[u].n};
                const int rc = enqueue_kquant_mfma_parts2(k0, j0, ty, k1, nseg - j0, ts[j0]->type, x, K, B, m->mm_part,
                                                          m->mm_part_floats);
                if (rc == ALJABR_ROCM_OK) return enqueue_slice_tail(*t, m->mm_part, slices, B, n_all);
                if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) return rc;
            }
            for (int i = 0, col = 0; i < nseg;) {
                int j = i + 1;
                while (j < nseg && ts[j]->type == ts[i]->type) ++j;
                KqOut k[3];
                int n = 0;
                for (int u = i; u < j; ++u) {
                    k[u - i] = KqOut{o[u].y, o[u].w, o[u].n};
                    n += o[u].n;
                }
                const int rc = enqueue_kquant_mfma_parts(k, j - i, x, K, ts[i]->type, B, m->mm_part,
                                                         m->mm_part_floats, n_all, col);
                // A refusal leaves nothing the fallback reads (it rewrites
                // every output).
                if (rc != ALJABR_ROCM_OK) return rc;
                col += n;
                i = j;
            }
            return enqueue_slice_tail(*t, m->mm_part, slices, B, n_all);
        }
        if (ty == ALJABR_ROCM_TYPE_NF4)
            return m->all_nf4 ? enqueue_nf4_mfma_multi(o, nseg, x, K, shift, B, false, m->mm_part, m->mm_part_floats, t,
                                                       xpacked)
                              : ALJABR_ROCM_ERR_UNSUPPORTED;
        if (!kquant_mfma_type(ty) || B > kquant_mfma_max_m(ty)) return ALJABR_ROCM_ERR_UNSUPPORTED;
        KqOut k[3];
        for (int i = 0; i < nseg; ++i) k[i] = KqOut{o[i].y, o[i].w, o[i].n};
        return enqueue_kquant_mfma_multi(k, nseg, x, K, ty, B, false, m->mm_part, m->mm_part_floats, t, xpacked);
    };
    // A residual tail defers RMSNorm's row scale only to a consumer that
    // takes a tail: matrices of one type, or K-quants the matrix cores take.
    auto takes_tail = [&](const T &a, const T &b, const T &c) {
        return (a.type == b.type && b.type == c.type) || (kq_ok(a) && kq_ok(b) && kq_ok(c));
    };
    hipLaunchKernelGGL(lengths_from_positions, dim3((B + 63) / 64), dim3(64), 0, s, m->kv_len, pos, B);
    if (m->tok_embed.type == ALJABR_ROCM_TYPE_F32)
        ALJ_TRY(enqueue_embed(m->x, reinterpret_cast<const float *>(m->tok_embed.w), tok, B, dim, c.vocab));
    else
        ALJ_TRY(enqueue_embed_typed(m->x, m->tok_embed.w, m->tok_embed.type, tok, B, dim, c.vocab));
    ALJ_MARK("embed", weight_bytes(m->tok_embed.type, B, dim, bs) + B * dim * f4);
    // With the GEMM tails, a residual tail may leave xb = x * norm_w without
    // RMSNorm's row scale, and the row-block sums of squares in tail_ssq: the
    // next GEMM's tail applies the scale to its products. A fallback that
    // consumes xb directly normalizes it first.
    bool xb_scaled = false;
    // Whether xb_pack / hb_pack hold xb / hb (the tail that wrote xb or hb
    // also wrote its A image).
    const bool packs = m->xb_pack && B <= 64;
    bool xb_packed = false, hb_packed = false;
    for (int l = 0; l < c.layers; ++l) {
        auto W = [&](const std::vector<T> &t) { return t[l].w; };
        auto S = [&](const std::vector<T> &t) { return t[l].s; };
        const float *attn_norm = m->attn_norm[l], *ffn_norm = m->ffn_norm[l];
        uint16_t *kc = m->k_cache + l * layer_cache;
        uint16_t *vc = m->v_cache + l * layer_cache;
        // Attention block: xb = RMSNorm(x); q, k, v = Wq/Wk/Wv xb; RoPE on
        // q and k; k and v appended to the cache.
        if (fused1) {
            const RowsOut qkv[3] = {{m->q, W(m->wq), S(m->wq), qd},
                                    {m->k, W(m->wk), S(m->wk), kvd},
                                    {m->v, W(m->wv), S(m->wv), kvd}};
            const int tq = m->wq[l].type, tk = m->wk[l].type, tv = m->wv[l].type;
            const RowsRope rope{pos, kc, vc, c.max_seq, hd, c.rope_base, m->rope_cs, c.n_kv_heads};
            // One launch per run of one type, the other segments left empty,
            // except Q4_K q and k beside a Q6_K v (a Q4_K_M model), which share
            // one launch of two row formats.
            const int types[3] = {tq, tk, tv};
            bool launched = false;
            if (tq == tk && tv != tq) {
                rc = enqueue_rows_mixed(tq, tv, qkv, m->x, attn_norm, c.eps, dim, kRowsRopeKV, &rope);
                if (rc != ALJABR_ROCM_ERR_UNSUPPORTED) {
                    if (rc != ALJABR_ROCM_OK) return rc;
                    launched = true;
                }
            }
            rc = ALJABR_ROCM_OK;
            for (int i = 0; i < 3 && rc == ALJABR_ROCM_OK && !launched;) {
                int j = i + 1;
                while (j < 3 && types[j] == types[i]) ++j;
                RowsOut part[3] = {qkv[0], qkv[1], qkv[2]};
                for (int u = 0; u < 3; ++u)
                    if (u < i || u >= j) part[u].n = 0;
                rc = enqueue_rows_fused(types[i], part, 3, m->x, attn_norm, c.eps, dim, shift, kRowsRopeKV, &rope);
                i = j;
            }
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                // A head size the epilogue does not take: plain launches, then
                // RoPE and the append (they rewrite whatever an earlier launch
                // of this loop stored, with the same values).
                for (int i = 0; i < 3;) {
                    int j = i + 1;
                    while (j < 3 && types[j] == types[i]) ++j;
                    ALJ_TRY(enqueue_rows_fused(types[i], qkv + i, j - i, m->x, attn_norm, c.eps, dim, shift, kRowsStore));
                    i = j;
                }
                ALJ_TRY(enqueue_rope_append(m->q, m->k, m->v, kc, vc, pos, B, nh, nkv, hd, c.max_seq, c.rope_base, m->rope_cs));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("qkv_rows_rmsnorm_rope_append",
                     weight_bytes(tq, qd, dim, bs) + weight_bytes(tk, kvd, dim, bs) + weight_bytes(tv, kvd, dim, bs) +
                         (2.0 * dim + qd) * f4 + 2.0 * kvd * 2.0);
        } else {
            // Every GEMM below writes its outputs (none accumulates into them).
            if (!tails || l == 0) {
                ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, attn_norm, B, dim, c.eps));
                ALJ_MARK("rmsnorm", (B * 2.0 * dim + dim) * f4);
            }
            // Q, K and V in one matrix-core launch where the shapes allow.
            const RowsOut qkv[3] = {{m->q, W(m->wq), S(m->wq), qd},
                                    {m->k, W(m->wk), S(m->wk), kvd},
                                    {m->v, W(m->wv), S(m->wv), kvd}};
            rc = ALJABR_ROCM_ERR_UNSUPPORTED;
            if (tails) {
                SliceTail t{};
                t.kind = kTailRopeAppend;
                t.out = m->q;
                t.kc = kc;
                t.vc = vc;
                t.pos = pos;
                t.nh = nh;
                t.nkv = nkv;
                t.head_dim = hd;
                t.cap = c.max_seq;
                t.base = c.rope_base;
                t.cs = m->rope_cs;
                t.ssq = xb_scaled ? m->tail_ssq : nullptr;
                t.norm_n = dim;
                t.eps = c.eps;
                const T *const qts[3] = {&m->wq[l], &m->wk[l], &m->wv[l]};
                rc = gemm_tail(qkv, qts, 3, m->xb, dim, &t, xb_packed ? m->xb_pack : nullptr);
                if (rc == ALJABR_ROCM_OK)
                    ALJ_MARK("qkv_gemm_rope_append", mm_bytes(m->wq[l], qd, dim, false) +
                                                         mm_bytes(m->wk[l], kvd, dim, false) +
                                                         mm_bytes(m->wv[l], kvd, dim, false) - 2.0 * B * dim * f4 -
                                                         B * 2.0 * kvd * f4 + B * 2.0 * kvd * 2.0);
            }
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                if (xb_scaled) ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, attn_norm, B, dim, c.eps));
                rc = m->all_nf4 && B >= 2 ? enqueue_nf4_mfma_multi(qkv, 3, m->xb, dim, shift, B, false, m->mm_part,
                                                                   m->mm_part_floats)
                                          : ALJABR_ROCM_ERR_UNSUPPORTED;
                if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                    float *const ys[3] = {m->q, m->k, m->v};
                    const T *const ts[3] = {&m->wq[l], &m->wk[l], &m->wv[l]};
                    const int ns[3] = {qd, kvd, kvd};
                    ALJ_TRY(mm_run(ys, ts, ns, 3, m->xb, dim));
                } else if (rc != ALJABR_ROCM_OK) {
                    return rc;
                }
                ALJ_MARK("qkv_gemm", mm_bytes(m->wq[l], qd, dim, false) + mm_bytes(m->wk[l], kvd, dim, false) +
                                         mm_bytes(m->wv[l], kvd, dim, false) - 2.0 * B * dim * f4);
                rc = enqueue_rope_append(m->q, m->k, m->v, kc, vc, pos, B, nh, nkv, hd, c.max_seq, c.rope_base,
                                         m->rope_cs);
                if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                    ALJ_TRY(enqueue_rope(m->q, pos, B, nh, hd, c.rope_base));
                    ALJ_TRY(enqueue_rope(m->k, pos, B, nkv, hd, c.rope_base));
                    ALJ_TRY(enqueue_kv_append(kc, m->k, pos, B, nkv, hd, c.max_seq));
                    ALJ_TRY(enqueue_kv_append(vc, m->v, pos, B, nkv, hd, c.max_seq));
                } else if (rc != ALJABR_ROCM_OK) {
                    return rc;
                }
                ALJ_MARK("rope_kv_append", B * (2.0 * qd + 2.0 * kvd) * f4 + B * 2.0 * kvd * 2.0);
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
        }
        AttnParams ap{};
        ap.out = m->att;
        ap.q = m->q;
        ap.k = kc;
        ap.v = vc;
        ap.mask = nullptr;
        ap.kv_len = m->kv_len;
        ap.B = B; ap.Hq = nh; ap.Hkv = nkv; ap.Sq = 1; ap.Sk = c.max_seq; ap.D = hd; ap.cap = c.max_seq;
        ap.scale = static_cast<float>(1.0 / sqrt(static_cast<double>(hd)));
        ap.causal = 0;
        ap.kv_f16 = 1;
        ap.scratch = m->attn_scratch;
        ap.scratch_bytes = m->attn_scratch_bytes;
        ap.scratch_only = 1;
        // With the Wo GEMM tail ahead, the attention kernels also write the
        // output's A image (no packing launch before the GEMM).
        ap.xpack = tails && packs && !fused1 ? m->att_pack : nullptr;
        rc = ap.xpack ? enqueue_attention(ap) : ALJABR_ROCM_ERR_UNSUPPORTED;
        const bool att_packed = rc == ALJABR_ROCM_OK;
        if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
            ap.xpack = nullptr;
            rc = enqueue_attention(ap);
        }
        ALJ_TRY(rc);
        ALJ_MARK("attention", keys * nkv * hd * 2.0 * 2.0 + B * 2.0 * qd * f4);
        // x += Wo att.
        if (fused1) {
            const RowsOut o = {m->x, W(m->wo), S(m->wo), dim};
            ALJ_TRY(enqueue_rows_fused(m->wo[l].type, &o, 1, m->att, nullptr, 0.0f, qd, shift, kRowsAdd));
            ALJ_MARK("wo_rows_add", mm_bytes(m->wo[l], dim, qd, true));
        } else {
            rc = ALJABR_ROCM_ERR_UNSUPPORTED;
            xb_scaled = false;
            if (tails) {
                // x += Wo att, then xb = x * the FFN norm with the row sums of
                // squares for the gate/up tail (RMSNorm's row scale), or the
                // full RMSNorm when gate and up cannot take a tail.
                const bool defer = takes_tail(m->w_gate[l], m->w_up[l], m->w_up[l]);
                SliceTail t{};
                t.kind = defer ? kTailResidualScale : kTailResidualNorm;
                t.out = m->x;
                t.xn = m->xb;
                t.norm_w = ffn_norm;
                t.eps = c.eps;
                t.ssq = m->tail_ssq;
                t.xpack = packs ? m->xb_pack : nullptr;
                const RowsOut o = {m->x, W(m->wo), S(m->wo), dim};
                const T *const ots[1] = {&m->wo[l]};
                rc = gemm_tail(&o, ots, 1, m->att, qd, &t, att_packed ? m->att_pack : nullptr);
                xb_packed = rc == ALJABR_ROCM_OK && packs;
                if (rc == ALJABR_ROCM_OK) {
                    xb_scaled = defer;
                    ALJ_MARK("wo_gemm_add_rmsnorm", mm_bytes(m->wo[l], dim, qd, true) + (B * dim + dim) * f4);
                }
            }
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                ALJ_TRY(mm(m->x, m->att, m->wo[l], qd, dim, true, m->xb));
                ALJ_MARK("wo_gemm_add", mm_bytes(m->wo[l], dim, qd, true));
                if (tails) {
                    ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, ffn_norm, B, dim, c.eps));
                    ALJ_MARK("rmsnorm", (B * 2.0 * dim + dim) * f4);
                }
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
        }
        // MLP: x += Wdown (silu(Wgate xb) * Wup xb), xb = RMSNorm(x).
        if (fused1) {
            const RowsOut gu[2] = {{m->hb, W(m->w_gate), S(m->w_gate), ffn},
                                   {nullptr, W(m->w_up), S(m->w_up), ffn}};
            const int tg = m->w_gate[l].type, tu = m->w_up[l].type;
            rc = tg == tu ? enqueue_rows_fused(tg, gu, 2, m->x, ffn_norm, c.eps, dim, shift, kRowsSwiGLU)
                          : ALJABR_ROCM_ERR_UNSUPPORTED;
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {     // mixed types, or a row count the paired waves do not divide
                const RowsOut gu2[2] = {{m->gate, W(m->w_gate), S(m->w_gate), ffn},
                                        {m->up, W(m->w_up), S(m->w_up), ffn}};
                if (tg == tu) {
                    ALJ_TRY(enqueue_rows_fused(tg, gu2, 2, m->x, ffn_norm, c.eps, dim, shift, kRowsStore));
                } else {
                    ALJ_TRY(enqueue_rows_fused(tg, gu2, 1, m->x, ffn_norm, c.eps, dim, shift, kRowsStore));
                    ALJ_TRY(enqueue_rows_fused(tu, gu2 + 1, 1, m->x, ffn_norm, c.eps, dim, shift, kRowsStore));
                }
                ALJ_TRY(enqueue_swiglu(m->hb, m->gate, m->up, ffn));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("gate_up_rows_rmsnorm_swiglu",
                     weight_bytes(tg, ffn, dim, bs) + weight_bytes(tu, ffn, dim, bs) + (2.0 * dim + ffn) * f4);
            const RowsOut d = {m->x, W(m->w_down), S(m->w_down), dim};
            ALJ_TRY(enqueue_rows_fused(m->w_down[l].type, &d, 1, m->hb, nullptr, 0.0f, ffn, shift, kRowsAdd));
            ALJ_MARK("down_rows_add", mm_bytes(m->w_down[l], dim, ffn, true));
        } else {
            if (!tails) {
                ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, ffn_norm, B, dim, c.eps));
                ALJ_MARK("rmsnorm", (B * 2.0 * dim + dim) * f4);
            }
            const RowsOut gu[2] = {{m->gate, W(m->w_gate), S(m->w_gate), ffn},
                                   {m->up, W(m->w_up), S(m->w_up), ffn}};
            rc = ALJABR_ROCM_ERR_UNSUPPORTED;
            if (tails) {
                SliceTail t{};
                t.kind = kTailSwiGLU;
                t.out = m->hb;
                t.n = ffn;
                t.ssq = xb_scaled ? m->tail_ssq : nullptr;
                t.norm_n = dim;
                t.eps = c.eps;
                t.xpack = packs ? m->hb_pack : nullptr;
                const T *const gts[2] = {&m->w_gate[l], &m->w_up[l]};
                rc = gemm_tail(gu, gts, 2, m->xb, dim, &t, xb_packed ? m->xb_pack : nullptr);
                hb_packed = rc == ALJABR_ROCM_OK && packs;
                if (rc == ALJABR_ROCM_OK)
                    ALJ_MARK("gate_up_gemm_swiglu", mm_bytes(m->w_gate[l], ffn, dim, false) +
                                                        mm_bytes(m->w_up[l], ffn, dim, false) - B * dim * f4 -
                                                        B * ffn * f4);
            }
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                if (xb_scaled) ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, ffn_norm, B, dim, c.eps));
                rc = m->all_nf4 && B >= 2 ? enqueue_nf4_mfma_multi(gu, 2, m->xb, dim, shift, B, false, m->mm_part,
                                                                   m->mm_part_floats)
                                          : ALJABR_ROCM_ERR_UNSUPPORTED;
                if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                    float *const ys[2] = {m->gate, m->up};
                    const T *const ts[2] = {&m->w_gate[l], &m->w_up[l]};
                    const int ns[2] = {ffn, ffn};
                    ALJ_TRY(mm_run(ys, ts, ns, 2, m->xb, dim));
                } else if (rc != ALJABR_ROCM_OK) {
                    return rc;
                }
                ALJ_MARK("gate_up_gemm", mm_bytes(m->w_gate[l], ffn, dim, false) +
                                             mm_bytes(m->w_up[l], ffn, dim, false) - B * dim * f4);
                ALJ_TRY(enqueue_swiglu(m->hb, m->gate, m->up, static_cast<long long>(B) * ffn));
                ALJ_MARK("swiglu", B * 3.0 * ffn * f4);
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            // x += Wdown hb; with the tails also xb = the next RMSNorm of x
            // (the next layer's attention norm, or the output norm).
            // Before the next layer: xb = x * its attention norm with the row
            // sums of squares (its Q/K/V tail applies the row scale); before
            // the output head: the full RMSNorm.
            const float *next_norm = l + 1 < c.layers ? m->attn_norm[l + 1] : m->out_norm;
            rc = ALJABR_ROCM_ERR_UNSUPPORTED;
            xb_scaled = false;
            if (tails) {
                const bool defer = l + 1 < c.layers && takes_tail(m->wq[l + 1], m->wk[l + 1], m->wv[l + 1]);
                SliceTail t{};
                t.kind = defer ? kTailResidualScale : kTailResidualNorm;
                t.out = m->x;
                t.xn = m->xb;
                t.norm_w = next_norm;
                t.eps = c.eps;
                t.ssq = m->tail_ssq;
                t.xpack = packs && defer ? m->xb_pack : nullptr;
                const RowsOut d = {m->x, W(m->w_down), S(m->w_down), dim};
                const T *const dts[1] = {&m->w_down[l]};
                rc = gemm_tail(&d, dts, 1, m->hb, ffn, &t, hb_packed ? m->hb_pack : nullptr);
                xb_packed = rc == ALJABR_ROCM_OK && packs && defer;
                if (rc == ALJABR_ROCM_OK) {
                    xb_scaled = defer;
                    ALJ_MARK("down_gemm_add_rmsnorm", mm_bytes(m->w_down[l], dim, ffn, true) + (B * dim + dim) * f4);
                }
            }
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                ALJ_TRY(mm(m->x, m->hb, m->w_down[l], ffn, dim, true, m->xb));
                ALJ_MARK("down_gemm_add", mm_bytes(m->w_down[l], dim, ffn, true));
                if (tails) {
                    ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, next_norm, B, dim, c.eps));
                    ALJ_MARK(l + 1 < c.layers ? "rmsnorm" : "final_rmsnorm", (B * 2.0 * dim + dim) * f4);
                }
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
        }
    }
    if (!tails) {
        ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, m->out_norm, B, dim, c.eps));
        ALJ_MARK("final_rmsnorm", (B * 2.0 * dim + dim) * f4);
    }
    ALJ_TRY(enqueue_matmul_typed(lg, m->xb, m->lm_head.w, m->lm_head.s, m->lm_head.type, bs, dim, c.vocab, B,
                                 m->mm_part, m->mm_part_floats));
    ALJ_MARK(m->lm_head.type == ALJABR_ROCM_TYPE_F16 ? "lm_head_f16" : "lm_head", mm_bytes(m->lm_head, c.vocab, dim, false));
    // The attention split buffer is free by now (stream order): the argmax's
    // chunk results go there.
    ALJ_TRY(enqueue_argmax(next, lg, B, c.vocab, m->attn_scratch, m->attn_scratch_bytes));
    ALJ_MARK("argmax", B * static_cast<double>(c.vocab) * f4);
#undef ALJ_MARK
#undef ALJ_TRY
    return ALJABR_ROCM_OK;
}

}  // namespace

extern "C" {

int aljabr_rocm_llama_decode(aljabr_rocm_llama *m, const void *tokens, const void *positions, int batch, void *logits,
                             void *next_tokens) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(m && tokens && positions && next_tokens, "model, tokens, positions and next_tokens are required");
    ALJ_REQUIRE(batch > 0 && batch <= m->cfg.max_batch, "batch %d outside [1, %d]", batch, m->cfg.max_batch);
    float *lg = logits ? static_cast<float *>(logits) : m->logits;
    const int rc = decode_step(m, static_cast<const int *>(tokens), static_cast<const int *>(positions), batch, lg,
                               static_cast<int *>(next_tokens), nullptr, nullptr);
    if (rc != ALJABR_ROCM_OK) return rc;
    return finish_launch("llama_decode");
}

int aljabr_rocm_llama_decode_graph(aljabr_rocm_llama *m, const void *tokens, const void *positions, int batch,
                                   void *logits, void *next_tokens) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(m && tokens && positions && next_tokens, "model, tokens, positions and next_tokens are required");
    ALJ_REQUIRE(batch > 0 && batch <= m->cfg.max_batch, "batch %d outside [1, %d]", batch, m->cfg.max_batch);
    hipStream_t s = current_stream();
    float *lg = logits ? static_cast<float *>(logits) : m->logits;
    const dim3 grid((batch + 63) / 64);
    hipLaunchKernelGGL(copy_i32_pairs, grid, dim3(64), 0, s, m->tok_in, static_cast<const int *>(tokens), m->pos_in,
                       static_cast<const int *>(positions), batch);
    aljabr_rocm_llama::Graph &g = m->graphs[static_cast<size_t>(batch)];
    if (g.exec && g.logits != lg) {              // another logits buffer: capture again
        (void)hipGraphExecDestroy(g.exec);
        g.exec = nullptr;
    }
    int rc;
    if (g.exec) {
        const hipError_t e = hipGraphLaunch(g.exec, s);
        if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipGraphLaunch: %s", hipGetErrorString(e));
    } else {
        // First step of this batch size: run it eagerly (which also sizes
        // every lazily allocated resource), then capture the same launches
        // without running them. The captured step reads the staged inputs,
        // so replays serve any tokens and positions.
        rc = decode_step(m, m->tok_in, m->pos_in, batch, lg, m->next_out, nullptr, nullptr);
        if (rc != ALJABR_ROCM_OK) return rc;
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipStreamBeginCapture: %s", hipGetErrorString(e));
        rc = decode_step(m, m->tok_in, m->pos_in, batch, lg, m->next_out, nullptr, nullptr);
        e = hipStreamEndCapture(s, &graph);
        if (rc != ALJABR_ROCM_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            g.exec = nullptr;
            return fail(ALJABR_ROCM_ERR_DEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
        }
        g.logits = lg;
    }
    hipLaunchKernelGGL(copy_i32_pairs, grid, dim3(64), 0, s, static_cast<int *>(next_tokens), m->next_out,
                       static_cast<int *>(nullptr), static_cast<const int *>(nullptr), batch);
    return finish_launch("llama_decode_graph");
}

int aljabr_rocm_llama_decode_profile(aljabr_rocm_llama *m, const void *tokens, const void *positions, int batch,
                                     void *logits, void *next_tokens, aljabr_rocm_kernel_stat *stats, int cap,
                                     int *count) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(m && tokens && positions && next_tokens && stats && count && cap > 0,
                "model, tokens, positions, next_tokens, stats and count are required");
    ALJ_REQUIRE(batch > 0 && batch <= m->cfg.max_batch, "batch %d outside [1, %d]", batch, m->cfg.max_batch);
    hipStream_t s = current_stream();
    std::vector<int> host_pos(static_cast<size_t>(batch));
    hipError_t e = hipMemcpyAsync(host_pos.data(), positions, sizeof(int) * batch, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "decode profile: positions: %s", hipGetErrorString(e));
    StepProfiler prof;
    int rc = prof.begin(s, static_cast<size_t>(m->cfg.layers) * 12 + 8);
    if (rc != ALJABR_ROCM_OK) return rc;
    float *lg = logits ? static_cast<float *>(logits) : m->logits;
    rc = decode_step(m, static_cast<const int *>(tokens), static_cast<const int *>(positions), batch, lg,
                     static_cast<int *>(next_tokens), &prof, host_pos.data());
    if (rc != ALJABR_ROCM_OK) return rc;
    e = hipEventSynchronize(prof.events[prof.used - 1]);
    if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "decode profile: %s", hipGetErrorString(e));
    int n = 0;
    for (size_t i = 0; i < prof.names.size(); ++i) {
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, prof.events[i], prof.events[i + 1]);
        if (e != hipSuccess) return fail(ALJABR_ROCM_ERR_DEVICE, "hipEventElapsedTime: %s", hipGetErrorString(e));
        int k = 0;
        while (k < n && std::strncmp(stats[k].name, prof.names[i], sizeof(stats[k].name)) != 0) ++k;
        if (k == n) {
            if (n == cap) continue;              // more groups than the caller has room for
            std::memset(&stats[n], 0, sizeof(stats[n]));
            std::strncpy(stats[n].name, prof.names[i], sizeof(stats[n].name) - 1);
            ++n;
        }
        stats[k].launches += 1;
        stats[k].us += 1000.0 * ms;
        stats[k].bytes += prof.bytes[i];
    }
    *count = n;
    return ALJABR_ROCM_OK;
}

}  // extern "C"
