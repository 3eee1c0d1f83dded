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
#include <algorithm>
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
    aljabr_rocm_llama_config cfg;
    std::vector<const void *> attn_norm, ffn_norm, wq, wk, wv, wo, wq_s, wk_s, wv_s, wo_s;
    std::vector<const void *> w_gate, w_up, w_down, w_gate_s, w_up_s, w_down_s;
    const void *tok_embed = nullptr, *out_norm = nullptr, *lm_head = nullptr;
    void *arena = nullptr;   // one allocation for the KV cache and activations
    uint16_t *k_cache = nullptr, *v_cache = nullptr;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float *gate = nullptr, *up = nullptr, *hb = nullptr, *logits = nullptr;
    int *kv_len = nullptr;
    int *tok_in = nullptr, *pos_in = nullptr, *next_out = nullptr;   // graph replays read and write these
    float *attn_scratch = nullptr;   // split-attention partials (owned: a captured graph keeps the address)
    size_t attn_scratch_bytes = 0;
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
                         ((B * c.vocab * 4 + 255) & ~size_t(255)) + ((B * 4 + 255) & ~size_t(255)) * 4 +
                         ((attention_scratch_bytes(c.max_batch, c.n_heads, 1, c.head_dim, c.max_seq) + 255) &
                          ~size_t(255)) + 256;
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
    m->graphs.resize(static_cast<size_t>(c.max_batch) + 1);
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
    for (auto &g : m->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
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
    // Bytes of one B-row NF4 product: weights once, activations in, outputs
    // out (read too when added into).
    auto mm_bytes = [&](long long N, long long K, bool add) {
        return nf4_w(N, K, bs) + B * (K + N * (add ? 2.0 : 1.0)) * f4;
    };
    const bool fused1 = B == 1 && m->rows_fused;
    hipLaunchKernelGGL(lengths_from_positions, dim3((B + 63) / 64), dim3(64), 0, s, m->kv_len, pos, B);
    ALJ_TRY(enqueue_embed(m->x, static_cast<const float *>(m->tok_embed), tok, B, dim, c.vocab));
    ALJ_MARK("embed", B * dim * 2.0 * f4);
    for (int l = 0; l < c.layers; ++l) {
        auto W = [&](const std::vector<const void *> &t) { return static_cast<const uint8_t *>(t[l]); };
        auto S = [&](const std::vector<const void *> &t) { return static_cast<const float *>(t[l]); };
        uint16_t *kc = m->k_cache + l * layer_cache;
        uint16_t *vc = m->v_cache + l * layer_cache;
        // Attention block: xb = RMSNorm(x); q, k, v = Wq/Wk/Wv xb; RoPE on
        // q and k; k and v appended to the cache.
        if (fused1) {
            const RowsOut qkv[3] = {{m->q, W(m->wq), S(m->wq_s), qd},
                                    {m->k, W(m->wk), S(m->wk_s), kvd},
                                    {m->v, W(m->wv), S(m->wv_s), kvd}};
            const RowsRope rope{pos, kc, vc, c.max_seq, hd, c.rope_base};
            rc = enqueue_nf4_rows_fused(qkv, 3, m->x, S(m->attn_norm), c.eps, dim, shift, kRowsRopeKV, &rope);
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {     // e.g. a head size that is not a power of two
                ALJ_TRY(enqueue_nf4_rows_fused(qkv, 3, m->x, S(m->attn_norm), c.eps, dim, shift, kRowsStore));
                ALJ_TRY(enqueue_rope_append(m->q, m->k, m->v, kc, vc, pos, B, nh, nkv, hd, c.max_seq, c.rope_base));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("qkv_rows_rmsnorm_rope_append",
                     nf4_w(qd + 2LL * kvd, dim, bs) + (2.0 * dim + qd) * f4 + 2.0 * kvd * 2.0);
        } else {
            const ZeroList z{{m->q, m->k, m->v},
                             {static_cast<long long>(B) * qd, static_cast<long long>(B) * kvd,
                              static_cast<long long>(B) * kvd}};
            ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, S(m->attn_norm), B, dim, c.eps, &z));
            ALJ_MARK("rmsnorm_clear", (B * 2.0 * dim + dim + B * (qd + 2.0 * kvd)) * f4);
            // Q, K and V in one matrix-core launch where the shapes allow.
            const RowsOut qkv[3] = {{m->q, W(m->wq), S(m->wq_s), qd},
                                    {m->k, W(m->wk), S(m->wk_s), kvd},
                                    {m->v, W(m->wv), S(m->wv_s), kvd}};
            rc = B >= 2 && B <= 64 ? enqueue_nf4_mfma_multi(qkv, 3, m->xb, dim, shift, B, true)
                                   : ALJABR_ROCM_ERR_UNSUPPORTED;
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                ALJ_TRY(mm(m->q, m->xb, m->wq[l], m->wq_s[l], dim, qd, false, nullptr));
                ALJ_TRY(mm(m->k, m->xb, m->wk[l], m->wk_s[l], dim, kvd, false, nullptr));
                ALJ_TRY(mm(m->v, m->xb, m->wv[l], m->wv_s[l], dim, kvd, false, nullptr));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("qkv_gemm", mm_bytes(qd + 2LL * kvd, dim, true));
        }
        if (!fused1) {
            rc = enqueue_rope_append(m->q, m->k, m->v, kc, vc, pos, B, nh, nkv, hd, c.max_seq, c.rope_base);
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                ALJ_TRY(enqueue_rope(m->q, pos, B, nh, hd, c.rope_base));
                ALJ_TRY(enqueue_rope(m->k, pos, B, nkv, hd, c.rope_base));
                ALJ_TRY(enqueue_kv_append(kc, m->k, pos, B, nkv, hd, c.max_seq));
                ALJ_TRY(enqueue_kv_append(vc, m->v, pos, B, nkv, hd, c.max_seq));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("rope_kv_append", B * (2.0 * qd + 2.0 * kvd) * f4 + B * 2.0 * kvd * 2.0);
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
        ALJ_TRY(enqueue_attention(ap));
        ALJ_MARK("attention", keys * nkv * hd * 2.0 * 2.0 + B * 2.0 * qd * f4);
        // x += Wo att.
        if (fused1) {
            const RowsOut o = {m->x, W(m->wo), S(m->wo_s), dim};
            ALJ_TRY(enqueue_nf4_rows_fused(&o, 1, m->att, nullptr, 0.0f, qd, shift, kRowsAdd));
            ALJ_MARK("wo_rows_add", mm_bytes(dim, qd, true));
        } else {
            ALJ_TRY(mm(m->x, m->att, m->wo[l], m->wo_s[l], qd, dim, true, m->xb));
            ALJ_MARK("wo_gemm_add", mm_bytes(dim, qd, true));
        }
        // MLP: x += Wdown (silu(Wgate xb) * Wup xb), xb = RMSNorm(x).
        if (fused1) {
            const RowsOut gu[2] = {{m->hb, W(m->w_gate), S(m->w_gate_s), ffn},
                                   {nullptr, W(m->w_up), S(m->w_up_s), ffn}};
            rc = enqueue_nf4_rows_fused(gu, 2, m->x, S(m->ffn_norm), c.eps, dim, shift, kRowsSwiGLU);
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {     // row count the paired waves do not divide
                const RowsOut gu2[2] = {{m->gate, W(m->w_gate), S(m->w_gate_s), ffn},
                                        {m->up, W(m->w_up), S(m->w_up_s), ffn}};
                ALJ_TRY(enqueue_nf4_rows_fused(gu2, 2, m->x, S(m->ffn_norm), c.eps, dim, shift, kRowsStore));
                ALJ_TRY(enqueue_swiglu(m->hb, m->gate, m->up, ffn));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("gate_up_rows_rmsnorm_swiglu", nf4_w(2LL * ffn, dim, bs) + (2.0 * dim + ffn) * f4);
            const RowsOut d = {m->x, W(m->w_down), S(m->w_down_s), dim};
            ALJ_TRY(enqueue_nf4_rows_fused(&d, 1, m->hb, nullptr, 0.0f, ffn, shift, kRowsAdd));
            ALJ_MARK("down_rows_add", mm_bytes(dim, ffn, true));
        } else {
            const ZeroList z{{m->gate, m->up, nullptr},
                             {static_cast<long long>(B) * ffn, static_cast<long long>(B) * ffn, 0}};
            ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, S(m->ffn_norm), B, dim, c.eps, &z));
            ALJ_MARK("rmsnorm_clear", (B * 2.0 * dim + dim + B * 2.0 * ffn) * f4);
            const RowsOut gu[2] = {{m->gate, W(m->w_gate), S(m->w_gate_s), ffn},
                                   {m->up, W(m->w_up), S(m->w_up_s), ffn}};
            rc = B >= 2 && B <= 64 ? enqueue_nf4_mfma_multi(gu, 2, m->xb, dim, shift, B, true)
                                   : ALJABR_ROCM_ERR_UNSUPPORTED;
            if (rc == ALJABR_ROCM_ERR_UNSUPPORTED) {
                ALJ_TRY(mm(m->gate, m->xb, m->w_gate[l], m->w_gate_s[l], dim, ffn, false, nullptr));
                ALJ_TRY(mm(m->up, m->xb, m->w_up[l], m->w_up_s[l], dim, ffn, false, nullptr));
            } else if (rc != ALJABR_ROCM_OK) {
                return rc;
            }
            ALJ_MARK("gate_up_gemm", mm_bytes(2LL * ffn, dim, true));
            ALJ_TRY(enqueue_swiglu(m->hb, m->gate, m->up, static_cast<long long>(B) * ffn));
            ALJ_MARK("swiglu", B * 3.0 * ffn * f4);
            ALJ_TRY(mm(m->x, m->hb, m->w_down[l], m->w_down_s[l], ffn, dim, true, m->xb));
            ALJ_MARK("down_gemm_add", mm_bytes(dim, ffn, true));
        }
    }
    ALJ_TRY(enqueue_rmsnorm(m->xb, m->x, static_cast<const float *>(m->out_norm), B, dim, c.eps));
    ALJ_MARK("final_rmsnorm", (B * 2.0 * dim + dim) * f4);
    ALJ_TRY(enqueue_matmul_gguf(lg, m->xb, static_cast<const uint8_t *>(m->lm_head), dim, c.vocab, ALJABR_ROCM_TYPE_F16,
                                B));
    ALJ_MARK("lm_head_f16", static_cast<double>(c.vocab) * dim * 2.0 + B * (static_cast<double>(dim) + c.vocab) * f4);
    ALJ_TRY(enqueue_argmax(next, lg, B, c.vocab));
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
