/*
 * aljabr_oracle.h - CPU restatement of Aljabr's quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path and
 * the timed CPU baseline in bench.py. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product (aljabr_amd/) never
 * links, loads or falls back to it.
 *
 * Every function names the reference file:line it restates. Paths are relative
 * to the andalus-ai/aljabr tree:
 *   STC = engine/safetensor/aljabr-safetensor-core/src/main/java/tech/kayys/aljabr/safetensor/core/tensor
 *   GRT = engine/gguf/aljabr-gguf-core/src/main/java/tech/kayys/aljabr/gguf/runtime
 *   GWR = engine/gguf/aljabr-gguf-core/src/main/java/tech/kayys/aljabr/gguf/writer
 *   GLD = engine/gguf/aljabr-gguf-core/src/main/java/tech/kayys/aljabr/gguf/loader
 *   CPU = backend/cpu/aljabr-backend-cpu/src/main/java/tech/kayys/aljabr/backend/cpu
 *   GJB = engine/gguf/aljabr-gguf-java/src/main/java/tech/kayys/aljabr/gguf/javabackend
 *
 * Parity status per function (what pins it) is listed beside each prototype.
 */
#ifndef ALJABR_ORACLE_H
#define ALJABR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */

/* GRT/GgufQuantTables.java:143-165 (f16ToF32Slow). Pinned: exhaustive 65536
 * comparison with the IEEE binary16 definition (numpy float16). */
float orc_f16_to_f32(uint16_t h);

/* GWR/GGUFWriter.java:360-387 (floatToHalfBits, round-half-up at bit 12).
 * Pinned: closed-form cases (exact halves, ties, subnormals, overflow). */
uint16_t orc_f32_to_f16_writer(float v);

/* java.lang.Math.round(float): nearest int, ties toward +inf, NaN -> 0,
 * saturating. Pinned: ties, negative ties, 0.49999997f. */
int32_t orc_java_round(float v);

/* ---- NF4 ---------------------------------------------------------------- */

/* STC/DequantizationKernel.java:23-28 */
extern const float ORC_NF4_TABLE[16];

/* STC/DequantizationKernel.java:84-102. Byte j holds element 2j in the high
 * nibble and 2j+1 in the low nibble; the scale index is (2j)/groupSize over the
 * flat element index. Pinned: closed form (one fp32 multiply) and the special
 * cases code 7 -> 0, codes 0/15 -> -/+absmax. */
void orc_nf4_dequant(const uint8_t *codes, const float *absmax, int64_t numel,
                     int32_t group_size, float *dst);

/* NF4 encoder. The reference's quantizer is absent from its tree (the BnB
 * adapter moved out), so this is build-defined: per-group absmax, value/absmax
 * rounded to the nearest codebook level, exact midpoint -> lower code.
 * PARITY UNPINNED against the reference; pinned only by the invariant
 * decode(encode(w)) == nearest level * absmax. */
void orc_nf4_quantize(const float *w, int64_t numel, int32_t group_size,
                      uint8_t *codes, float *absmax);

/* NF4 linear y[m,n] = sum_k x[m,k] * W[n,k], W = dequantized NF4 (fp32),
 * restating STC/AccelOps.java:392-463 (JIT dequant then an fp32 GEMV/GEMM).
 * The GEMV itself is Apple Accelerate there (third-party, absent); this uses a
 * 16-lane fp32 dot per row. Pinned against a float64 brute force in tests. */
void orc_nf4_matvec(const uint8_t *codes, const float *absmax, int32_t group_size,
                    const float *x, int64_t n_rows, int64_t k_cols, int32_t m,
                    float *y, int threads);

/* ---- GGUF Q4_0 / Q8_0 --------------------------------------------------- */

/* GWR/GGUFWriter.java:179-209 (encodeQ4_0, quantize4, maxAbs). numel % 32 == 0. */
void orc_q4_0_quantize(const float *w, int64_t numel, uint8_t *out);
/* GWR/GGUFWriter.java:163-177 (encodeQ8_0). numel % 32 == 0. */
void orc_q8_0_quantize(const float *w, int64_t numel, uint8_t *out);

/* GRT/GgufBlockDequantizer.java:33-37,366-416 (low nibble -> j, high -> j+16,
 * (q-8)*d + 0.0f). Pinned: GgufQ32Test/GgufNibFx known answers. */
void orc_q4_0_dequant(const uint8_t *blocks, int64_t numel, float *dst);
/* GRT/GgufBlockDequantizer.java:231-265 (int8 * d). Pinned: GgufQ8Test. */
void orc_q8_0_dequant(const uint8_t *blocks, int64_t numel, float *dst);

/* GRT/GgufQ32RawDot.java:34-67,342-349,428-463: four block accumulators, four
 * intra-block lane partials, same fp32 operation order. */
float orc_q4_0_dot_row(const uint8_t *row, int32_t columns, const float *x);
/* GRT/GgufQ8RawDot.java:138-185,784-830 (scalar path). */
float orc_q8_0_dot_row(const uint8_t *row, int32_t columns, const float *x);

/* Row-parallel matvec / batched matvec: y[m*N + n] = dot(row n, x[m*K ...]).
 * Row chunks = min(rows, 2*threads) as GRT/GgufParallelConfig.java:64-73. */
void orc_q4_0_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads);
void orc_q8_0_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads);

/* ---- GGUF K-quants Q4_K / Q6_K ------------------------------------------ */

/* GRT/GgufKBlockDequantizer.java:32-90 + GRT/GgufKQuantLayout.java:38-70
 * (144-byte super-blocks: f16 d, f16 dMin, 12 bytes of 6-bit scale/min codes,
 * 128 bytes of nibbles; d*sc*q - dMin*min, a zero min code contributing 0).
 * numel % 256 == 0. Pinned: GgufQ4KPrepTest/GgufQ4KMixTest/GgufKZeroMinTest
 * known answers, the GgufQ4CalcFx lane-order rows, and round trips of
 * independently packed scale/min codes (tests/test_oracle.py). */
void orc_q4_k_dequant(const uint8_t *blocks, int64_t numel, float *dst);
/* GRT/GgufKBlockDequantizer.java:320-425 (210-byte super-blocks: ql[128],
 * qh[64], int8 scales[16], f16 d; (q6 - 32) * d * scale[e / 16]). Pinned:
 * GgufQ6KPrepTest known answers, GgufQ6LaneFx lane-order rows, per-16 scale
 * closed form. */
void orc_q6_k_dequant(const uint8_t *blocks, int64_t numel, float *dst);
/* GRT/GgufQ4RawDot.java:38-148 (d1*dot1 + d2*dot2 - dMin*min*sum(x)). */
float orc_q4_k_dot_row(const uint8_t *row, int32_t columns, const float *x);
/* GRT/GgufQ6RawDot.java:33-133,403-514. */
float orc_q6_k_dot_row(const uint8_t *row, int32_t columns, const float *x);
void orc_q4_k_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads);
void orc_q6_k_matvec(const uint8_t *w, const float *x, int64_t n_rows,
                     int64_t k_cols, int32_t m, float *y, int threads);
/* y = cap * tanh(y / cap): MTLC/aljabr_metal_kernel_source.m:111-118. */
void orc_softcap(float *y, int64_t n, float cap);

/* fp16 rows (LM head): GRT/GgufDenseRows.java:70-90. */
void orc_f16_matvec(const uint16_t *w, const float *x, int64_t n_rows,
                    int64_t k_cols, int32_t m, float *y, int threads);

/* ---- attention ---------------------------------------------------------- */

/* CPU/CpuBackend.java:1546-1748 (attentionGqa + computeAttentionGroup):
 * Q[B,Hq,Sq,D], K/V[B,Hkv,Sk,D] fp32, optional additive mask [Sq,Sk], causal
 * bottom-right alignment, online softmax with double denominators and double
 * weighted values. Returns 0, or -2 on invalid shapes/mask (the reference's
 * IllegalArgumentException). Pinned: CpuBatchedAttentionTest and
 * CpuBackendStorageTest known answers. */
int orc_attention_gqa(const float *q, const float *k, const float *v,
                      const float *mask, int64_t b, int64_t hq, int64_t hkv,
                      int64_t sq, int64_t sk, int64_t d, int causal,
                      float *out, int threads);
/* Paged-KV attention, MTLC/aljabr_metal_attention.m:146-355 (CPU bridge path). */
int orc_paged_attention(const float *q, const float *kc, const float *vc, const int32_t *block_table,
                        const int32_t *context_lens, int32_t b_n, int32_t t_n, int32_t h_n, int32_t hkv,
                        int32_t d, int32_t block_size, int32_t max_blocks, float scale, int32_t is_causal,
                        int32_t query_start_pos, int32_t sliding_window, float soft_cap, float *out);
/* Prefill (FA4) attention, MTLC/aljabr_metal_fa4.m:111-115,466-530: Q/out
 * [B,T,H,D], K/V [B,S,H_kv,D] float32; row t sees keys [lo, hi) with hi = S or,
 * causal, min(max(S - T, 0) + t + 1, S); lo = 0, or max(hi - window, 0) for
 * window > 0 (an extension the Metal entry point does not have). Returns 0,
 * or -1 for a shape it rejects. */
int orc_fa4_attention(const float *q, const float *k, const float *v, int32_t b_n, int32_t t_n, int32_t s_n,
                      int32_t h_n, int32_t hkv, int32_t d, float scale, int32_t is_causal, float soft_cap,
                      int32_t window, float *out);

/* ---- decode-step element-wise ops --------------------------------------- */

/* GLD/tensor/GGUFVectorOps.java:211-234 */
void orc_rmsnorm(const float *x, const float *w, float *out, int32_t len, float eps);
/* GLD/tensor/GGUFVectorOps.java:383-440 (split-half, fp32 table). */
void orc_rope(float *x, int32_t n_heads, int32_t head_dim, int32_t pos, float base);
/* GLD/tensor/GGUFVectorOps.java:333-338 */
void orc_swiglu(const float *gate, const float *up, float *dst, int32_t len);
/* GLD/tensor/GGUFVectorOps.java:302-317 */
void orc_softmax(float *a, int32_t len);

/* ---- Llama-shaped decode step ------------------------------------------- */

/* GJB/GgufDecodeAttentionExecution.java:68-104: single-token GQA attention
 * over a position-major cache window ([position][cache_head_stride], KV head
 * h at h * head_dim), positions [start_position, sequence_length) visible;
 * `scores` holds sequence_length - start_position floats. The decode step's
 * attention. Pinned by GgufDecodeAttentionExecutionTest.java:15-66 (GQA head
 * mapping {15,15,150,150}, window {20,200}, {25}) and against the dense
 * attention oracle (tests/test_oracle.py). */
void orc_decode_attention(const float *query, float *output, float *scores, const float *key_cache,
                          const float *value_cache, int32_t cache_head_stride, int32_t kv_heads,
                          int32_t query_heads, int32_t head_dim, int32_t sequence_length,
                          int32_t start_position, float scale);

typedef struct orc_llama_cfg {
    int32_t layers, dim, ffn, n_heads, n_kv_heads, head_dim, vocab, max_seq;
    int32_t nf4_group;
    int32_t kv_f16;      /* 1: K/V rounded to binary16 (nearest-even) when stored */
    float rope_base, eps;
} orc_llama_cfg;

/* Weights for one model, all host pointers. Per-layer arrays are indexed by
 * layer. Projection weights are NF4 [out, in]; the LM head is fp16
 * [vocab, dim]; embeddings fp32 [vocab, dim]. */
typedef struct orc_llama_weights {
    const float *tok_embed;
    const float *const *attn_norm;
    const float *const *ffn_norm;
    const uint8_t *const *wq, *const *wk, *const *wv, *const *wo;
    const float *const *wq_s, *const *wk_s, *const *wv_s, *const *wo_s;
    const uint8_t *const *w_gate, *const *w_up, *const *w_down;
    const float *const *w_gate_s, *const *w_up_s, *const *w_down_s;
    const float *out_norm;
    const uint16_t *lm_head;
} orc_llama_weights;

/* One decode position for one sequence, GJB/GgufDecodePass.java:297-505 and
 * GJB/GgufLogitsProcessor.java:26-48: the KV caches are fp32 [layers][max_seq]
 * [n_kv_heads*head_dim]. Writes logits[vocab] and the final hidden state
 * x[dim]; returns the greedy token. */
int32_t orc_llama_decode(const orc_llama_cfg *cfg, const orc_llama_weights *w,
                         int32_t token, int32_t pos, float *k_cache,
                         float *v_cache, float *logits, float *hidden,
                         int threads);

/* One weight tensor of a typed model: data, type (0 F32, 1 F16, 2 Q4_0,
 * 8 Q8_0, 12 Q4_K, 14 Q6_K, 100 NF4 with absmax and group). */
typedef struct orc_tensor {
    const void *data;
    const float *absmax;
    int32_t type;
    int32_t group;
} orc_tensor;
typedef struct orc_llama_typed {
    orc_tensor tok_embed;
    const float *const *attn_norm, *const *ffn_norm;
    const orc_tensor *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float *out_norm;
    orc_tensor lm_head;
} orc_llama_typed;
/* GJB/GgufDecodePass.java:183-592 over per-tensor GGUF types: the same step
 * as orc_llama_decode (which runs through it) with each matvec dispatched on
 * its type and the embedding row decoded from its type. Its parts are pinned
 * on their own (per-type matvec and dequant, RMSNorm/RoPE/SwiGLU KATs,
 * orc_decode_attention's KATs); the composition is pinned by an independent
 * full-sequence causal forward in numpy at every position and by closed forms
 * (zero Wo and W_down; one layer at position 0) in tests/test_oracle.py. */
int32_t orc_llama_decode_typed(const orc_llama_cfg *cfg, const orc_llama_typed *w,
                               int32_t token, int32_t pos, float *k_cache,
                               float *v_cache, float *logits, float *hidden,
                               int threads);

/* ---- Metal whole-step decode (registered layers) ------------------------ */

/* One layer as aljabr_metal_register_decode_layer records it
 * (MTLC/aljabr_metal_matvec_api.m:3348-3425): absent wk / wv have data NULL
 * (a layer without wk attends to the cache of its kv_layer chain's owner;
 * wk without wv uses the raw K projection as V); rope_freqs NULL: no
 * frequency divisors. */
typedef struct orc_step_layer {
    orc_tensor wq, wk, wv, wo, gate, up, down;
    int32_t kv_layer, n0, n1, n2, wo_k, wo_n, ffn, n_heads, n_kv_heads, head_dim;
    float freq_base;
    int32_t is_swa;
    float out_scale, attn_scale;
    int32_t has_post_attn_norm, has_post_ffn_norm, has_q_norm, has_k_norm, has_unit_v_norm;
    const float *rope_freqs;
    int32_t rope_freqs_len;
} orc_step_layer;

/* The registered model: norm slots as aljabr_metal_register_norm_buffer
 * takes them (0 post-attention, 1 FFN, 2 post-FFN, 3 attention norm, each
 * [layers][dim]; 4 Q and 5 K head norms [layers][max head_dim]; NULL: not
 * registered), fp32 KV caches per layer [max_seq][kv_stride[l]] (NULL:
 * none), the output norm and projection (out_w.data NULL: no logits) with
 * softcap `cap` (<= 0: none), the token embedding (embd_rows rows of the
 * model width, multiplied by embd_scale) and the FFN activation kind (1
 * SiLU, 2 tanh GELU). */
typedef struct orc_step_model {
    int32_t layers;
    const orc_step_layer *layer;
    const float *norm[6];
    float *const *k_cache, *const *v_cache;
    const int32_t *kv_stride;
    const float *out_norm;
    orc_tensor out_w;
    int32_t out_k, out_n;
    float cap;
    orc_tensor embd;
    int32_t embd_rows;
    float embd_scale;
    int32_t activation;
} orc_step_model;

/* aljabr_metal_decode_step / _token at one position
 * (MTLC/aljabr_metal_matvec_api.m:3574-4083): x = x_in (token < 0) or the
 * embedding row of `token`; per layer attention norm, Q/K/V, K-as-V copy,
 * Q/K head norms, unit V norm, RoPE with divisors, cache store, attention over
 * the owner's cache (sliding window on SWA layers, scale attn_scale or 1 with
 * head norms or 1/sqrt(D)), Wo, post-attention norm, residual, FFN norm,
 * gated FFN, post-FFN norm, residual and output scale; then output norm,
 * logits and softcap. Writes the final residual to x[dim] and logits[out_n];
 * returns the greedy token, or the reference's negative codes (-3 required
 * norms missing, -4 no KV owner, -5 KV geometry mismatch, -6 bad K-as-V or
 * token). Pinned by tests/test_oracle_step.py: equal to orc_llama_decode_typed
 * with the Gemma features off, and to an independent full-sequence numpy
 * forward with every feature on, with planted mistakes caught. */
int32_t orc_step_decode(const orc_step_model *m, int32_t pos, int32_t window, float eps, int32_t token,
                        const float *x_in, float *x, float *logits, int threads);

/* binary32 -> binary16 -> binary32 with round-to-nearest-even (IEEE). */
float orc_round_f16(float v);

/* ---- deterministic generator -------------------------------------------- */

/* SplitMix64 -> Box-Muller (build-defined): out[i] = mean + std * N(0,1). */
void orc_fill_normal(uint64_t seed, float mean, float std, float *out, int64_t n);
/* SplitMix64 -> uniform integers in [0, bound). */
void orc_fill_uniform_int(uint64_t seed, int32_t bound, int32_t *out, int64_t n);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
