// llama.hip - device-resident Llama-style decode step over NF4 weights.
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
#include <cstring>
#include <new>
#include <vector>

#include "device.hpp"
#include "internal.hpp"
#include "kernels.hpp"

namespace aljabr {

namespace {

__global__ void lengths_from_positions(int *__restrict__ len, const int *__restrict__ pos, int n) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) len[i] = pos[i] + 1;
}

}  // namespace
}  // namespace aljabr

struct aljabr_rocm_llama {
    aljabr_rocm_llama_config cfg;
    std::vector<const void *> attn_norm, ffn_norm, wq, wk, wv, wo, wq_s, wk_s, wv_s, wo_s;
    std::vector<const void *> w_gate, w_up, w_down, w_gate_s, w_up_s, w_down_s;
    const void *tok_embed = nullptr, *out_norm = nullptr, *lm_head = nullptr;
    void *arena = nullptr;   // one allocation for the KV cache and activations
    uint16_t *k_cache = nullptr, *v_cache = nullptr;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float *gate = nullptr, *up = nullptr, *hb = nullptr, *logits = nullptr;
    int *kv_len = nullptr;
    bool rows_fused = false;   // batch-1 layers as four fused NF4 launches (shapes and alignment allow it)
};

using namespace aljabr;

namespace {

template <class T>
T *carve(char *&cursor, size_t count) {
    T *p = reinterpret_cast<T *>(cursor);
    cursor += (count * sizeof(T) + 255) & ~static_cast<size_t>(255);
    return p;
}

bool copy_table(std::vector<const void *> &dst, const void *const *src, int n) {
    if (!src) return false;
    dst.assign(src, src + n);
    for (const void *p : dst)
        if (!p) return false;
    return true;
}

}  // namespace

extern "C" {

int aljabr_rocm_llama_create(const aljabr_rocm_llama_config *cfg, const aljabr_rocm_llama_weights *w,
                             aljabr_rocm_llama **out) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(cfg && w && out, "cfg, weights and out must be non-null");
    *out = nullptr;
    const aljabr_rocm_llama_config &c = *cfg;
    ALJ_REQUIRE(c.layers > 0 && c.dim > 0 && c.ffn > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.head_dim > 0 &&
                    c.vocab > 0 && c.max_seq > 0 && c.max_batch > 0 && c.nf4_block > 0,
                "llama config dimensions must be positive");
    ALJ_REQUIRE(c.n_heads % c.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    ALJ_REQUIRE(c.head_dim % 2 == 0 && c.nf4_block % 2 == 0, "head_dim and nf4_block must be even");
    ALJ_REQUIRE(c.rope_base > 1.0f && c.eps >= 0.0f, "rope_base must exceed 1 and eps be non-negative");
    ALJ_REQUIRE(w->tok_embed && w->out_norm && w->lm_head, "embedding, output norm and LM head are required");

    aljabr_rocm_llama *m = new (std::nothrow) aljabr_rocm_llama();
    if (!m) return fail(ALJABR_ROCM_ERR_BUFFER, "out of host memory");
    m->cfg = c;
    const int L = c.layers;
    bool ok = copy_table(m->attn_norm, w->attn_norm, L) && copy_table(m->ffn_norm, w->ffn_norm, L) &&
              copy_table(m->wq, w->wq, L) && copy_table(m->wk, w->wk, L) && copy_table(m->wv, w->wv, L) &&
              copy_table(m->wo, w->wo, L) && copy_table(m->wq_s, w->wq_absmax, L) &&
              copy_table(m->wk_s, w->wk_absmax, L) && copy_table(m->wv_s, w->wv_absmax, L) &&
              copy_table(m->wo_s, w->wo_absmax, L) && copy_table(m->w_gate, w->w_gate, L) &&
              copy_table(m->w_up, w->w_up, L) && copy_table(m->w_down, w->w_down, L) &&
              copy_table(m->w_gate_s, w->w_gate_absmax, L) && copy_table(m->w_up_s, w->w_up_absmax, L) &&
              copy_table(m->w_down_s, w->w_down_absmax, L);
    if (!ok) {
        delete m;
        return fail(ALJABR_ROCM_ERR_BAD_ARGUMENT, "every per-layer weight pointer must be non-null");
    }
    m->tok_embed = w->tok_embed;
    m->out_norm = w->out_norm;
    m->lm_head = w->lm_head;

    const size_t B = static_cast<size_t>(c.max_batch);
    const size_t kvd = static_cast<size_t>(c.n_kv_heads) * c.head_dim;
    const size_t qd = static_cast<size_t>(c.n_heads) * c.head_dim;
    const size_t cache_elems = static_cast<size_t>(L) * B * kvd * c.max_seq;
    const size_t bytes = 2 * ((cache_elems * 2 + 255) & ~size_t(255)) +
                         ((B * c.dim * 4 + 255) & ~size_t(255)) * 2 + ((B * qd * 4 + 255) & ~size_t(255)) * 2 +
                         ((B * kvd * 4 + 255) & ~size_t(255)) * 2 + ((B * c.ffn * 4 + 255) & ~size_t(255)) * 3 +
                         ((B * c.vocab * 4 + 255) & ~size_t(255)) + ((B * 4 + 255) & ~size_t(255)) + 256;
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
    // Batch-1 fusion needs every K a multiple of 2048 (at most 16384), a
    // power-of-two block of at least 32 and 16-byte aligned weights and norms.
    const int qd_i = c.n_heads * c.head_dim;
    const int shift = log2_exact(c.nf4_block);
    auto k_ok = [](int k) { return k % 2048 == 0 && k / 2048 >= 1 && k / 2048 <= 8; };
    bool fused = k_ok(c.dim) && k_ok(qd_i) && k_ok(c.ffn) && shift >= 5;
    for (int l = 0; l < L && fused; ++l)
        for (const auto *t : {&m->attn_norm, &m->ffn_norm, &m->wq, &m->wk, &m->wv, &m->wo, &m->w_gate, &m->w_up,
                              &m->w_down})
            fused = fused && aligned((*t)[l], 16);
    m->rows_fused = fused;
    *out = m;
    return ALJABR_ROCM_OK;
}

int aljabr_rocm_llama_destroy(aljabr_rocm_llama *m) {
    if (!m) return ALJABR_ROCM_OK;
    ALJ_CHECK_READY();
    if (m->arena) (void)hipFree(m->arena);
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

int aljabr_rocm_llama_decode(aljabr_rocm_llama *m, const void *tokens, const void *positions, int batch, void *logits,
                             void *next_tokens) {
    ALJ_CHECK_READY();
    ALJ_REQUIRE(m && tokens && positions && next_tokens, "model, tokens, positions and next_tokens are required");
    const aljabr_rocm_llama_config &c = m->cfg;
    ALJ_REQUIRE(batch > 0 && batch <= c.max_batch, "batch %d outside [1, %d]", batch, c.max_batch);
    const int *pos = static_cast<const int *>(positions);
    const int *tok = static_cast<const int *>(tokens);
    const int B = batch, dim = c.dim, hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv_heads;
    const int qd = nh * hd, kvd = nkv * hd, ffn = c.ffn, bs = c.nf4_block;
    const int shift = log2_exact(bs);
    const size_t layer_cache = static_cast<size_t>(c.max_batch) * kvd * c.max_seq;
    float *lg = logits ? static_cast<float *>(logits) : m->logits;
    int rc;
#define ALJ_TRY(expr)                           \
    do {                                        \
        rc = (expr);                            \
        if (rc != ALJABR_ROCM_OK) return rc;    \
    } while (0)
    hipStream_t s = current_stream();
    // y = x . W^T (y cleared beforehand) or, with `residual`, y += x . W^T for
    // B rows. The matrix cores' K-slices add straight into y in both cases;
    // elsewhere y is written, or the products go to `tmp` and one add follows.
    auto mm = [&](float *y, const float *x, const void *w, const void *sc, int K, int N, bool residual,
                  float *tmp) -> int {
        const uint8_t *wq = static_cast<const uint8_t *>(w);
        const float *ws = static_cast<const float *>(sc);
        if (B >= 2 && B <= 64 && shift >= 0) {
            const int r = enqueue_nf4_mfma(y, x, wq, ws, K, N, shift, B, true);
            if (r != ALJABR_ROCM_ERR_UNSUPPORTED) return r;
        }
        if (!residual) return enqueue_matmul_nf4(y, x, wq, ws, K, N, bs, B);
        const int r = enqueue_matmul_nf4(tmp, x, wq, ws, K, N, bs, B);
        if (r != ALJABR_ROCM_OK) return r;
        return enqueue_add(y, tmp, static_cast<long long>(B) * N);
    };
    const bool fused1 = B == 1 && m->rows_fused;
    hipLaunchKernelGGL(lengths_from_positions, dim3((B + 63) / 64), dim3(64), 0, s, m->kv_len, pos, B);
    ALJ_TRY(enqueue_embed(m->x, static_cast<const float *>(m->tok_embed), tok, B, dim, c.vocab));
    for (int l = 0; l < c.layers; ++l) {
        auto W = [&](const std::vector<const void *> &t) { return static_cast<const uint8_t *>(t[l]); };
        auto S = [&](const std::vector<const void *> &t) { return static_cast<const float *>(t[l]); };
        uint16_t *kc = m->k_cache + l * layer_cache;
        uint16_t *vc = m->v_cache + l * layer_cache;
        // Attention block: xb = RMSNorm(x); q, k, v = Wq/Wk/Wv xb.
        if (fused1) {
            const RowsOut qkv[3] = {{m->q, W(m->wq), S(m->wq_s), qd, 0},
                                    {m->k, W(m->wk), S(m->wk_s), kvd, 0},
                                    {m->v, W(m->wv), S(m->wv_s), kvd, 0}};
            ALJ_TRY(enqueue_nf4_rows_fused(qkv, 3, m->x, nullptr, S(m->attn_norm), c.eps, dim, shift, kRowsNorm, 0));
        } else {
            const ZeroList z{{m->q, m->k, m->v},
                             {static_cast<long long>(B) * qd, static_cast<long long>(B) * kvd,
                              static_cast<long long>(B) * kvd}};
            ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, S(m->attn_norm), B, dim, c.eps, &z));
            ALJ_TRY(mm(m->q, m->xb, m->wq[l], m->wq_s[l], dim, qd, false, nullptr));
            ALJ_TRY(mm(m->k, m->xb, m->wk[l], m->wk_s[l], dim, kvd, false, nullptr));
            ALJ_TRY(mm(m->v, m->xb, m->wv[l], m->wv_s[l], dim, kvd, false, nullptr));
        }
        rc = enqueue_rope_append(m->q, m->k, m->v, kc, vc, pos, B, nh, nkv, hd, c.max_seq, c.rope_base);
        if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
            ALJ_TRY(enqueue_rope(m->q, pos, B, nh, hd, c.rope_base));
            ALJ_TRY(enqueue_rope(m->k, pos, B, nkv, hd, c.rope_base));
            ALJ_TRY(enqueue_kv_append(kc, m->k, pos, B, nkv, hd, c.max_seq));
            ALJ_TRY(enqueue_kv_append(vc, m->v, pos, B, nkv, hd, c.max_seq));
        } else if (rc != ALJABR_ROCM_OK) {
            return rc;
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
        ALJ_TRY(enqueue_attention(ap));
        // x += Wo att.
        if (fused1) {
            const RowsOut o = {m->x, W(m->wo), S(m->wo_s), dim, 0};
            ALJ_TRY(enqueue_nf4_rows_fused(&o, 1, m->att, nullptr, nullptr, 0.0f, qd, shift, kRowsPlain, 1));
        } else {
            ALJ_TRY(mm(m->x, m->att, m->wo[l], m->wo_s[l], qd, dim, true, m->xb));
        }
        // MLP: x += Wdown (silu(Wgate xb) * Wup xb), xb = RMSNorm(x).
        if (fused1) {
            const RowsOut gu[2] = {{m->gate, W(m->w_gate), S(m->w_gate_s), ffn, 1},
                                   {m->up, W(m->w_up), S(m->w_up_s), ffn, 0}};
            ALJ_TRY(enqueue_nf4_rows_fused(gu, 2, m->x, nullptr, S(m->ffn_norm), c.eps, dim, shift, kRowsNorm, 0));
            const RowsOut d = {m->x, W(m->w_down), S(m->w_down_s), dim, 0};
            ALJ_TRY(enqueue_nf4_rows_fused(&d, 1, m->gate, m->up, nullptr, 0.0f, ffn, shift, kRowsMul, 1));
        } else {
            const ZeroList z{{m->gate, m->up, nullptr},
                             {static_cast<long long>(B) * ffn, static_cast<long long>(B) * ffn, 0}};
            ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, S(m->ffn_norm), B, dim, c.eps, &z));
            ALJ_TRY(mm(m->gate, m->xb, m->w_gate[l], m->w_gate_s[l], dim, ffn, false, nullptr));
            ALJ_TRY(mm(m->up, m->xb, m->w_up[l], m->w_up_s[l], dim, ffn, false, nullptr));
            ALJ_TRY(enqueue_swiglu(m->hb, m->gate, m->up, static_cast<long long>(B) * ffn));
            ALJ_TRY(mm(m->x, m->hb, m->w_down[l], m->w_down_s[l], ffn, dim, true, m->xb));
        }
    }
    ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, static_cast<const float *>(m->out_norm), B, dim, c.eps));
    ALJ_TRY(enqueue_matmul_gguf(lg, m->xb, static_cast<const uint8_t *>(m->lm_head), dim, c.vocab, ALJABR_ROCM_TYPE_F16,
                                B));
    ALJ_TRY(enqueue_argmax(static_cast<int *>(next_tokens), lg, B, c.vocab));
#undef ALJ_TRY
    return finish_launch("llama_decode");
}

}  // extern "C"
