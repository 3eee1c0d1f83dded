/*
 * aljabr_rocm.h - C ABI of Aljabr's MI355X (gfx950) quantized-inference path.
 *
 * This is the drop-in boundary a Java provider binds through the JDK Foreign
 * Function & Memory API (SymbolLookup.libraryLookup + Linker.downcallHandle),
 * exactly as MetalBinding binds libaljabr_metal
 * (backend/metal/aljabr-backend-metal/src/main/java/tech/kayys/aljabr/metal/binding/MetalBinding.java:205-230,1799-1818).
 * Every entry point takes plain pointers and sizes and returns an int status.
 *
 * Pointers named C/A/B/out/Q/K/V/x/y are DEVICE pointers (from
 * aljabr_rocm_alloc or any HIP allocation on the initialised device); host
 * pointers appear only in the memcpy and info calls. Reference citations are
 * relative to the andalus-ai/aljabr tree; MTLC = backend/metal/aljabr-backend-metal/src/main/cpp/metal.
 *
 * Execution model. Work is enqueued on the calling thread's stream (one
 * library-owned HIP stream per thread, or the stream set by
 * aljabr_rocm_set_stream). With sync mode on (the default, matching the
 * reference contract that every native call returns after completion) each
 * compute call waits for its stream before returning and reports device
 * errors; with sync mode off calls are stream-ordered and
 * aljabr_rocm_synchronize() waits. Concurrent calls from different threads use
 * different streams and never share scratch memory.
 */
#ifndef ALJABR_ROCM_H
#define ALJABR_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: the Metal ABI's codes (MTLC/aljabr_metal_matvec_api.m:506-520,
 * MTLC/aljabr_metal_matvec_dispatch.m:644-662) plus a HIP runtime error. ---- */
#define ALJABR_ROCM_OK 0
#define ALJABR_ROCM_ERR_NOT_INITIALIZED (-1)
#define ALJABR_ROCM_ERR_BAD_ARGUMENT (-2)   /* bad dimensions, null or misaligned pointer */
#define ALJABR_ROCM_ERR_UNSUPPORTED (-3)    /* no kernel for this type/shape ("missing pipeline") */
#define ALJABR_ROCM_ERR_BUFFER (-4)         /* allocation or copy failure */
#define ALJABR_ROCM_ERR_DEVICE (-5)         /* HIP runtime / launch / execution error */

/* ---- weight type ids: GGML ids as used by aljabr_metal_matvec_tb_batch
 * (MTLC/aljabr_metal_matvec_api.m:1091-1100; engine/gguf/aljabr-gguf-core/.../core/GgmlType.java:12,17),
 * plus NF4, which has no GGML id (the reference's DType has no NF4 entry). ---- */
#define ALJABR_ROCM_TYPE_F32 0
#define ALJABR_ROCM_TYPE_F16 1
#define ALJABR_ROCM_TYPE_Q4_0 2
#define ALJABR_ROCM_TYPE_Q8_0 8
#define ALJABR_ROCM_TYPE_Q4_K 12
#define ALJABR_ROCM_TYPE_Q6_K 14
#define ALJABR_ROCM_TYPE_NF4 100

/* ======================================================================== */
/* lifecycle and device                                                      */
/* ======================================================================== */

/* Select device `ordinal`, check it is gfx950 (this library carries gfx950
 * code objects only) and create the context. Idempotent for the same ordinal.
 * Replaces the Metal init that MetalComputeBackend runs at session open
 * (backend/metal/.../MetalComputeBackend.java:127-145). */
int aljabr_rocm_init(int ordinal);
/* Release every library-owned stream and scratch buffer. Idempotent. */
int aljabr_rocm_shutdown(void);
int aljabr_rocm_is_initialized(void);
/* Number of visible HIP devices (0 when no GPU); does not need init. */
int aljabr_rocm_device_count(int *count);

typedef struct aljabr_rocm_device_info {
    char name[256];
    char arch[64];             /* e.g. "gfx950:sramecc+:xnack-" */
    uint64_t total_bytes;
    uint64_t free_bytes;
    int32_t compute_units;
    int32_t wavefront_size;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int32_t l2_bytes;
    int32_t runtime_version;
    int32_t driver_version;
} aljabr_rocm_device_info;

/* Fills DeviceDescriptor's fields (spi/aljabr-spi-core/.../DeviceDescriptor.java:10-37). */
int aljabr_rocm_device_info_get(int ordinal, aljabr_rocm_device_info *info);

/* Thread-local message for the last non-zero status on this thread. */
const char *aljabr_rocm_last_error(void);
/* Library version as major*10000 + minor*100 + patch. */
int aljabr_rocm_version(void);

/* ======================================================================== */
/* streams and memory (TensorStorage lifetime: one alloc <-> one free)        */
/* ======================================================================== */

/* Bind the calling thread to an existing hipStream_t (NULL: back to the
 * library's own stream for this thread). */
int aljabr_rocm_set_stream(void *hip_stream);
int aljabr_rocm_get_stream(void **hip_stream);
/* 1 (default): compute calls return after completion; 0: stream-ordered. Per thread. */
int aljabr_rocm_set_sync_mode(int synchronous);
int aljabr_rocm_synchronize(void);
/* Bytes of device scratch the library holds for the calling thread's stream
 * (grown on demand by calls that bring no buffer of their own; never taken
 * while the stream is being captured). No counterpart in the reference: a
 * diagnostic for callers that capture or budget device memory. */
int aljabr_rocm_stream_scratch_bytes(size_t *bytes);
/* Reads `bytes` (a multiple of 16) of device memory at `src` once, with
 * `workgroups` workgroups of 256 lanes, and writes nothing to `sink` in
 * practice (one 4-byte word at most). No counterpart in the reference: the
 * plain streaming read the batch-1 matvec kernels are measured against. */
int aljabr_rocm_stream_read_probe(const void *src, size_t bytes, void *sink, int workgroups);

/* Device allocation backing RocmDeviceStorage; the final TensorStorage.release()
 * maps to aljabr_rocm_free (plugins/ml/aljabr-tensor/.../memory/TensorStorage.java:21-41). */
int aljabr_rocm_alloc(size_t bytes, void **device_ptr);
int aljabr_rocm_free(void *device_ptr);
/* ComputeBackend.copyFromHost (plugins/ml/aljabr-tensor/.../backend/ComputeBackend.java:151-162). */
int aljabr_rocm_memcpy_h2d(void *device_dst, const void *host_src, size_t bytes);
int aljabr_rocm_memcpy_d2h(void *host_dst, const void *device_src, size_t bytes);
int aljabr_rocm_memcpy_d2d(void *device_dst, const void *device_src, size_t bytes);
/* Byte fill with a kernel (never a memset node, so callers may capture it). */
int aljabr_rocm_fill_u8(void *device_dst, int value, size_t bytes);

/* ======================================================================== */
/* quantized matvec / small-M GEMM: C[m][n] = sum_k A[m][k] * W[n][k]         */
/* W is [N,K] row-major ("transposed right", MTLJ/MetalComputeBackend.java:435-470). */
/* ======================================================================== */

/* NF4, batch 1. B_packed: N*K/2 bytes, byte j = (code[2j] << 4) | code[2j+1];
 * absmax: fp32 per blockSize elements over the flat [N,K] index.
 * Replaces aljabr_metal_matvec_tb_nf4 (MTLC/aljabr_metal_matvec_api.h:59-61). */
int aljabr_rocm_matvec_tb_nf4(void *C, const void *A, const void *B_packed,
                              const void *absmax, int K, int N, int blockSize);
/* GGUF Q4_0 blocks {f16 d; u8 qs[16]} (no Metal counterpart; the GGUF CPU
 * runtime's GgufQ32RawDot.dotRowQ4_0 rows, engine/gguf/.../runtime/GgufQ32RawDot.java:34-67). */
int aljabr_rocm_matvec_tb_q4_0(void *C, const void *A, const void *B, int K, int N);
/* GGUF Q8_0 blocks {f16 d; i8 qs[32]}; replaces aljabr_metal_matvec_tb_q8_0
 * (MTLC/aljabr_metal_matvec_api.h:55). */
int aljabr_rocm_matvec_tb_q8_0(void *C, const void *A, const void *B, int K, int N);
/* fp16 rows (LM head); replaces aljabr_metal_matvec_tb_half (MTLC/aljabr_metal_matvec_api.h:32-33). */
int aljabr_rocm_matvec_tb_half(void *C, const void *A, const void *B, int K, int N);
/* GGUF K-quants, rows of K/256 super-blocks: Q4_K 144-byte blocks {f16 d;
 * f16 dmin; u8 scales[12]; u8 qs[128]}, Q6_K 210-byte blocks {u8 ql[128];
 * u8 qh[64]; i8 scales[16]; f16 d} (engine/gguf/.../runtime/GgufKBlockDequantizer.java:32-90,320-425).
 * K must be a multiple of 256 (-2 otherwise); A and B 16-byte aligned.
 * Replace aljabr_metal_matvec_tb_q4_k / _q6_k (MTLC/aljabr_metal_matvec_api.h:48-55). */
int aljabr_rocm_matvec_tb_q4_k(void *C, const void *A, const void *B, int K, int N);
int aljabr_rocm_matvec_tb_q6_k(void *C, const void *A, const void *B, int K, int N);
/* The same with the output soft cap C[n] = cap * tanh(C[n] / cap) when cap > 0
 * (MTLC/aljabr_metal_matvec_api.m:448-505; aljabr_softcap_kernel,
 * MTLC/aljabr_metal_kernel_source.m:111-118). */
int aljabr_rocm_matvec_tb_q4_k_softcap(void *C, const void *A, const void *B, int K, int N, float cap);
int aljabr_rocm_matvec_tb_q6_k_softcap(void *C, const void *A, const void *B, int K, int N, float cap);

/* A[batchSize][K] fp32 -> C[batchSize][N] fp32 with W read once per call.
 * type: ALJABR_ROCM_TYPE_{Q4_0,Q8_0,Q4_K,Q6_K,F16}. Replaces aljabr_metal_matvec_tb_batch
 * (MTLC/aljabr_metal_matvec_api.h:93-94). batchSize < 16 runs the
 * wavefront-reduction kernels, batchSize >= 16 the MFMA kernels. */
int aljabr_rocm_matvec_tb_batch(void *C, const void *A, const void *B, int K,
                                int N, int type, int batchSize);
/* NF4 variant of the above (the Metal ABI has no NF4 batch entry). */
int aljabr_rocm_matvec_tb_batch_nf4(void *C, const void *A, const void *B_packed,
                                    const void *absmax, int K, int N,
                                    int blockSize, int batchSize);

/* ======================================================================== */
/* codecs                                                                    */
/* ======================================================================== */

/* Decode `numel` weights to fp32, bit-exact with the reference decoders:
 * NF4 STC/DequantizationKernel.java:84-102 (absmax/blockSize used), Q4_0
 * GgufBlockDequantizer.java:33-37,403-416 (+0.0f), Q8_0 :231-265, Q4_K and Q6_K
 * GgufKBlockDequantizer.java:32-90,320-425 (numel % 256 == 0), F16
 * GgufQuantTables.java:143-165. STC = engine/safetensor/aljabr-safetensor-core/.../core/tensor. */
int aljabr_rocm_dequantize(void *dst_f32, const void *src, const void *absmax,
                           long long numel, int type, int blockSize);
/* Encode fp32 weights. Q4_0/Q8_0 follow GGUFWriter.encodeQ4_0/encodeQ8_0
 * bit-for-bit (engine/gguf/aljabr-gguf-core/.../writer/GGUFWriter.java:163-209,360-387);
 * NF4 uses per-block absmax and nearest-level codes (the reference's NF4
 * quantizer is not in its tree). F16 uses the writer's half rounding. */
int aljabr_rocm_quantize(void *dst, void *absmax_out, const void *src_f32,
                         long long numel, int type, int blockSize);

/* ======================================================================== */
/* attention                                                                 */
/* ======================================================================== */

/* Dense GQA attention with CpuBackend.attentionGqa semantics
 * (backend/cpu/.../CpuBackend.java:1546-1748): Q[B,Hq,Sq,D] fp32,
 * K/V[B,Hkv,Sk,D] (kvType F32 or F16), optional additive mask [Sq,Sk] fp32
 * (NULL for none; NaN/+inf entries are rejected with -2), bottom-right causal
 * alignment, scale = 1/sqrt(D) when scale <= 0. out[B,Hq,Sq,D] fp32.
 * Split-K online softmax; D must be 64 or 128 (else -3). */
int aljabr_rocm_attention_gqa(void *out, const void *Q, const void *K, const void *V,
                              const void *mask, int B, int Hq, int Hkv, int Sq,
                              int Sk, int D, int kvType, float scale, int causal);

/* No counterpart in the reference: aljabr_rocm_attention_gqa for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results, mask must be
 * NULL (-3 otherwise). The split partials live in a 32 MiB device array each
 * GPU holds until the process ends, four 8 MiB slots: B*Hq*Sq*2*(D+2)*4 bytes
 * must fit in a slot (-2 otherwise), and the split count is lowered to what it
 * holds. No device or host allocation happens (the calling thread's stream is
 * the one set with aljabr_rocm_set_stream; without one, a thread's first call
 * to the library creates its stream). Each slot serves one stream at a time:
 * calls on one stream are ordered by it, up to four streams per GPU run
 * concurrently, and a fifth stream waits for the device to drain before it
 * takes the least recently used slot (so it must not be called while another
 * stream of the process is being captured). */
int aljabr_rocm_attention_gqa_noalloc(void *out, const void *Q, const void *K, const void *V,
                                      const void *mask, int B, int Hq, int Hkv, int Sq,
                                      int Sk, int D, int kvType, float scale, int causal);

/* Paged-KV attention with the argument lists of the Metal bridge
 * (MTLC/aljabr_metal_attention.h:14-36, semantics of aljabr_metal_attention_impl,
 * MTLC/aljabr_metal_attention.m:146-355): Q and out [B,T,H,D] fp32; K/V caches
 * fp32 [num_blocks][H_kv][block_size][D]; key j of sequence b is row j % block_size of
 * block block_table[b*max_blocks + j/block_size]; context_lens[b] keys per sequence
 * (<= 0: zero output). Query t sits at query_start_pos + t, or at
 * context_len - T + t when causal with no window and query_start_pos == 0; causal
 * keys reach up to that position, a sliding window > 0 starts at position - window
 * + 1. soft_cap > 0 caps scores as soft_cap * tanh(score / soft_cap); weights are
 * exp(s - max) / (sum + 1e-9). Status -1 when H is not a multiple of H_kv (as
 * Metal), -2 for non-positive sizes, a context longer than max_blocks blocks or a
 * negative block index. All pointers are device pointers; the call checks the
 * table on the device and waits for that check. */
int aljabr_rocm_paged_attention(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                const int *block_table, const int *context_lens, int B, int T, int H,
                                int D, int block_size, int max_blocks, float scale, int is_causal,
                                float soft_cap);
int aljabr_rocm_paged_attention_windowed(void *out, const void *Q, const void *K_cache,
                                         const void *V_cache, const int *block_table,
                                         const int *context_lens, int B, int T, int H, int D,
                                         int block_size, int max_blocks, float scale, int is_causal,
                                         int query_start_pos, int sliding_window, float soft_cap);
int aljabr_rocm_paged_attention_gqa(void *out, const void *Q, const void *K_cache, const void *V_cache,
                                    const int *block_table, const int *context_lens, int B, int T,
                                    int H, int H_kv, int D, int block_size, int max_blocks,
                                    float scale, int is_causal, float soft_cap);
int aljabr_rocm_paged_attention_gqa_windowed(void *out, const void *Q, const void *K_cache,
                                             const void *V_cache, const int *block_table,
                                             const int *context_lens, int B, int T, int H, int H_kv,
                                             int D, int block_size, int max_blocks, float scale,
                                             int is_causal, int query_start_pos, int sliding_window,
                                             float soft_cap);

/* ======================================================================== */
/* Several matrices over one input (replaces MTLC/aljabr_metal_matvec_api.h: */
/* 83-120): device pointers; types F32 0, F16 1, Q4_0 2, Q8_0 8, Q4_K 12,    */
/* Q6_K 14. Matrices of one type share a launch.                             */
/* ======================================================================== */

/* C_i[N_i] = B_i[N_i][K] . A[K] for i = 0, 1 (the gate/up pair). */
int aljabr_rocm_matvec_tb_pair(void *C0, void *C1, const void *A, const void *B0, const void *B1, int K, int N0,
                               int N1, int type0, int type1);
/* The same for three matrices (Q/K/V). */
int aljabr_rocm_matvec_tb_triple(void *C0, void *C1, void *C2, const void *A, const void *B0, const void *B1,
                                 const void *B2, int K, int N0, int N1, int N2, int type0, int type1, int type2);
/* Batched: A [batchSize][K], C_i [batchSize][N_i]. */
int aljabr_rocm_matvec_tb_triple_batch(void *C0, void *C1, void *C2, const void *A, const void *B0, const void *B1,
                                       const void *B2, int K, int N0, int N1, int N2, int type0, int type1, int type2,
                                       int batchSize);
/* outDown[dim] = W_down[dim][ffnDim] . (act(W_gate . inA) * (W_up . inA)),
 * act = SiLU (g / (1 + e^-g), 0 below -20, g above 20) or, for
 * activationKind 2, the tanh GELU (0 below -10, g above 10); a non-finite
 * product becomes 0 (aljabr_metal_kernel_source.m:72-108). inA and outDown
 * are device pointers here (the Metal call copies host arrays). */
int aljabr_rocm_ffn_gated_fused(void *outDown, const void *inA, const void *gateW, const void *upW, const void *downW,
                                int dim, int ffnDim, int typeGate, int typeUp, int typeDown, int activationKind);
/* Batched: inA, outDown [batchSize][dim]. */
int aljabr_rocm_ffn_gated_fused_batch(void *outDown, const void *inA, const void *gateW, const void *upW,
                                      const void *downW, int dim, int ffnDim, int typeGate, int typeUp, int typeDown,
                                      int activationKind, int batchSize);

/* ======================================================================== */
/* safetensors files (replaces engine/safetensor/aljabr-safetensor-loader/   */
/* .../SafetensorHeaderParser.java:13-160 and the NF4 path of                */
/* aljabr-safetensor-bridge/.../AccelWeightBridge.java:184-222)              */
/* ======================================================================== */

/* dtype ids, in the order of the reference's SafetensorDType enum */
#define ALJABR_ROCM_ST_BF16 0
#define ALJABR_ROCM_ST_F16 1
#define ALJABR_ROCM_ST_F32 2
#define ALJABR_ROCM_ST_F64 3
#define ALJABR_ROCM_ST_F8_E4M3 4
#define ALJABR_ROCM_ST_F8_E5M2 5
#define ALJABR_ROCM_ST_I8 6
#define ALJABR_ROCM_ST_I16 7
#define ALJABR_ROCM_ST_I32 8
#define ALJABR_ROCM_ST_I64 9
#define ALJABR_ROCM_ST_U8 10
#define ALJABR_ROCM_ST_U16 11
#define ALJABR_ROCM_ST_U32 12
#define ALJABR_ROCM_ST_U64 13
#define ALJABR_ROCM_ST_BOOL 14

typedef struct aljabr_rocm_safetensors aljabr_rocm_safetensors;

/* Maps `path` read-only and parses it: u64 little-endian header length (at
 * most 100 MiB), JSON {name: {dtype, shape, data_offsets}, "__metadata__":
 * {string: string}}; every range inside the file, equal to shape x dtype
 * size, none overlapping. -2 with a message for a malformed file. */
int aljabr_rocm_safetensors_open(const char *path, aljabr_rocm_safetensors **out);
int aljabr_rocm_safetensors_close(aljabr_rocm_safetensors *f);
int aljabr_rocm_safetensors_tensor_count(const aljabr_rocm_safetensors *f, int64_t *count);
int aljabr_rocm_safetensors_find_tensor(const aljabr_rocm_safetensors *f, const char *name, int64_t *index);
/* Name (NUL-terminated, truncated to name_cap), dtype id, rank, dims[8]
 * (unused entries 0) and byte size of tensor `index`; outputs may be null. */
int aljabr_rocm_safetensors_tensor_info(const aljabr_rocm_safetensors *f, int64_t index, char *name, int name_cap,
                                        int32_t *dtype, int32_t *n_dims, int64_t *dims, uint64_t *bytes);
/* Host pointer to the tensor's bytes inside the mapping (valid until close). */
int aljabr_rocm_safetensors_tensor_data(const aljabr_rocm_safetensors *f, int64_t index, const void **host_data);
/* Value of a "__metadata__" key into `value` (value_cap bytes, NUL-terminated). */
int aljabr_rocm_safetensors_meta(const aljabr_rocm_safetensors *f, const char *key, char *value, int value_cap);
/* The NF4 weight "<base_name>.qweight" (U8 [N, K/2], two codes a byte, high
 * nibble first) + "<base_name>.scales" (F32, one absmax per 128 weights)
 * copied to two new device buffers the caller frees with aljabr_rocm_free;
 * rows = N, cols = K, block_size = 128, the layout every NF4 entry point
 * takes (AccelWeightBridge.attachQuantizationMetadata). */
int aljabr_rocm_safetensors_upload_nf4(const aljabr_rocm_safetensors *f, const char *base_name, void **codes,
                                       void **absmax, int64_t *rows, int64_t *cols, int32_t *block_size);

/* ======================================================================== */
/* Prefill attention (replaces MTLC/aljabr_metal_fa4.m:253-257,542-556)      */
/* ======================================================================== */

/* out[B,T,H,D] = softmax(scale * Q K^T) V per head, Q [B,T,H,D], K/V
 * [B,S,H_kv,D] device pointers, all fp32, H % H_kv == 0 (query head h reads
 * KV head h / (H / H_kv)). With is_causal, row t sees keys
 * [0, min(max(S - T, 0) + t + 1, S)), the bottom-right limit of
 * aljabr_metal_fa4.m:111-115; soft_cap > 0 maps each kept score to
 * cap * tanh(score / cap) first. use_bf16 is accepted and ignored: results
 * are fp32-accurate. Flash-style on the matrix cores for D = 64 and 128
 * (16-byte aligned pointers), a generic kernel for other D <= 256.
 * Replaces aljabr_metal_fa4_attention (same argument order). */
int aljabr_rocm_fa4_attention(void *output, const void *query, const void *key, const void *value, int B, int T,
                              int S, int H, int H_kv, int D, float scale, int is_causal, int use_bf16,
                              float soft_cap);
/* The same with a sliding window: row t sees keys [max(hi - window, 0), hi)
 * where hi is the limit above (window <= 0: no window). No Metal
 * counterpart; it serves the windowed prefill the GGUF runner otherwise runs
 * on the CPU (GJB/GgufPrefillAttentionExecution.java:33-78). */
int aljabr_rocm_fa4_attention_windowed(void *output, const void *query, const void *key, const void *value, int B,
                                       int T, int S, int H, int H_kv, int D, float scale, int is_causal,
                                       float soft_cap, int window);
/* 1: the fused path is available (aljabr_metal_fa4_sdpa_available). */
int aljabr_rocm_fa4_sdpa_available(void);
/* 0: no reduced-precision bf16 arithmetic is offered (aljabr_metal_fa4_bf16_available). */
int aljabr_rocm_fa4_bf16_available(void);

/* ======================================================================== */
/* decode-step element-wise ops (fp32)                                       */
/* ======================================================================== */

/* out[r] = x[r] * 1/sqrt(mean(x[r]^2)+eps) * w, rows of `len`
 * (GGUFVectorOps.rmsNorm, engine/gguf/.../loader/tensor/GGUFVectorOps.java:211-234). */
int aljabr_rocm_rmsnorm(void *out, const void *x, const void *w, int rows, int len, float eps);
/* In-place split-half RoPE over `rows` token rows of nHeads*headDim values,
 * position pos[r] (device int32) for row r (GGUFVectorOps.java:383-440). */
int aljabr_rocm_rope(void *x, const void *positions, int rows, int nHeads,
                     int headDim, float base);
/* dst = silu(gate) * up (GGUFVectorOps.java:333-338). */
int aljabr_rocm_swiglu(void *dst, const void *gate, const void *up, long long n);
/* a += b (GGUFVectorOps.addInPlace, GGUFVectorOps.java:108-116). */
int aljabr_rocm_add_inplace(void *a, const void *b, long long n);
/* out[r] = argmax(x[r]) over `cols` (first index on ties), rows of fp32. */
int aljabr_rocm_argmax(void *out_i32, const void *x, int rows, int cols);

/* ======================================================================== */
/* Llama-shaped NF4 decode step (whole step device-resident)                 */
/* ======================================================================== */

typedef struct aljabr_rocm_llama_config {
    int32_t layers, dim, ffn, n_heads, n_kv_heads, head_dim, vocab, max_seq;
    int32_t nf4_block;      /* NF4 absmax block size */
    int32_t max_batch;      /* sequences decoded together */
    float rope_base, eps;
} aljabr_rocm_llama_config;

/* Device pointers to one model's weights. Projection weights are NF4 [out,in]
 * codes + fp32 absmax; norms fp32; token embedding fp32 [vocab,dim]; LM head
 * fp16 [vocab,dim]. Per-layer pointer arrays are HOST arrays of `layers`
 * device pointers. */
typedef struct aljabr_rocm_llama_weights {
    const void *tok_embed;
    const void *const *attn_norm, *const *ffn_norm;
    const void *const *wq, *const *wk, *const *wv, *const *wo;
    const void *const *wq_absmax, *const *wk_absmax, *const *wv_absmax, *const *wo_absmax;
    const void *const *w_gate, *const *w_up, *const *w_down;
    const void *const *w_gate_absmax, *const *w_up_absmax, *const *w_down_absmax;
    const void *out_norm;
    const void *lm_head;
} aljabr_rocm_llama_weights;

typedef struct aljabr_rocm_llama aljabr_rocm_llama;

/* Create a decode session: copies the pointer tables and allocates the fp16 KV
 * cache [layers][max_batch][n_kv_heads][max_seq][head_dim] and activations.
 * Weights stay owned by the caller. (GgufDecodePass + KVCache,
 * engine/gguf/aljabr-gguf-java/.../GgufDecodePass.java:183-592.) */
int aljabr_rocm_llama_create(const aljabr_rocm_llama_config *cfg,
                             const aljabr_rocm_llama_weights *w,
                             aljabr_rocm_llama **out);
int aljabr_rocm_llama_destroy(aljabr_rocm_llama *model);
/* One greedy decode step for `batch` sequences: tokens[b] (device int32) at
 * positions[b] (device int32, < max_seq). Writes logits[batch][vocab] fp32 (may
 * be NULL) and next_tokens[batch] (device int32). */
int aljabr_rocm_llama_decode(aljabr_rocm_llama *model, const void *tokens,
                             const void *positions, int batch, void *logits,
                             void *next_tokens);
/* One weight tensor of a typed session: device data and its
 * ALJABR_ROCM_TYPE_*; for NF4 also the fp32 absmax array and block size (0 or
 * the config's nf4_block). Rows of K elements must be whole blocks of the
 * type (32 for Q4_0/Q8_0, 256 for Q4_K/Q6_K). */
typedef struct aljabr_rocm_tensor {
    const void *data;
    const void *absmax;
    int32_t type;
    int32_t block_size;
} aljabr_rocm_tensor;

/* Weights of a typed session (the GGUF runner's per-tensor types, e.g. a
 * Q4_K_M file: Q4_K projections with Q6_K attn_v/ffn_down/output). Per-layer
 * arrays are HOST arrays of `layers` entries; norms are fp32 device vectors.
 * tok_embed: F32, F16, Q4_0, Q8_0, Q4_K or Q6_K; projections and lm_head:
 * those or NF4. */
typedef struct aljabr_rocm_llama_tensors {
    aljabr_rocm_tensor tok_embed;                       /* [vocab, dim] */
    const void *const *attn_norm, *const *ffn_norm;     /* [dim] fp32 */
    const aljabr_rocm_tensor *wq, *wk, *wv, *wo;        /* [n_heads*head_dim|n_kv*head_dim, dim], [dim, n_heads*head_dim] */
    const aljabr_rocm_tensor *w_gate, *w_up, *w_down;   /* [ffn, dim], [ffn, dim], [dim, ffn] */
    const void *out_norm;                               /* [dim] fp32 */
    aljabr_rocm_tensor lm_head;                         /* [vocab, dim] */
} aljabr_rocm_llama_tensors;

/* A decode session over typed weights (any mix per matrix), the GGUF decode
 * runner's contract (GgufDecodePass over per-tensor GgmlTypes,
 * engine/gguf/aljabr-gguf-java/.../GgufDecodePass.java:183-592, registered the
 * way aljabr_metal_register_decode_layer takes per-matrix types,
 * MTLC/aljabr_metal_matvec_api.h:244-282). All-NF4 weights take the same fused
 * paths as aljabr_rocm_llama_create. Weights stay owned by the caller; every
 * decode entry point below accepts the session. */
int aljabr_rocm_llama_create_typed(const aljabr_rocm_llama_config *cfg,
                                   const aljabr_rocm_llama_tensors *w,
                                   aljabr_rocm_llama **out);

/* ---- GGUF files ---------------------------------------------------------- */

/* A GGUF file mapped read-only and parsed (header, metadata, tensor table),
 * as the reference's GGUFParser reads it (engine/gguf/aljabr-gguf-core/.../
 * loader/GGUFParser.java:18-63): versions 2 and 3, data at general.alignment
 * (default 32). Host only: needs no device and no aljabr_rocm_init. Malformed
 * or truncated files give -2, tensor types it cannot size -3. */
typedef struct aljabr_rocm_gguf aljabr_rocm_gguf;
int aljabr_rocm_gguf_open(const char *path, aljabr_rocm_gguf **out);
int aljabr_rocm_gguf_close(aljabr_rocm_gguf *g);
int aljabr_rocm_gguf_tensor_count(const aljabr_rocm_gguf *g, int64_t *n);
int aljabr_rocm_gguf_find_tensor(const aljabr_rocm_gguf *g, const char *name, int64_t *index);
/* dims[4] in GGUF order (dims[0] = row length); offset from the file start. */
int aljabr_rocm_gguf_tensor_info(const aljabr_rocm_gguf *g, int64_t index, char *name, int name_cap,
                                 int32_t *type, int32_t *n_dims, int64_t *dims, uint64_t *offset,
                                 uint64_t *bytes);
/* Host pointer into the mapping (valid until aljabr_rocm_gguf_close). */
int aljabr_rocm_gguf_tensor_data(const aljabr_rocm_gguf *g, int64_t index, const void **host_data);
/* Metadata by key: integers and bools (arrays: their length), numbers, strings. */
int aljabr_rocm_gguf_meta_int(const aljabr_rocm_gguf *g, const char *key, int64_t *value);
int aljabr_rocm_gguf_meta_float(const aljabr_rocm_gguf *g, const char *key, double *value);
int aljabr_rocm_gguf_meta_string(const aljabr_rocm_gguf *g, const char *key, char *buf, int cap);

/* A typed decode session from a Llama-family GGUF file: the configuration
 * from {arch}.block_count / embedding_length / feed_forward_length /
 * attention.head_count(_kv) / attention.key_length / rope.freq_base /
 * attention.layer_norm_rms_epsilon (max_seq <= 0: {arch}.context_length), the
 * tensors token_embd, blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output,
 * ffn_norm, ffn_gate, ffn_up, ffn_down}, output_norm and output (absent: tied
 * to token_embd), uploaded once into device memory the session owns. The
 * reference path: GgufLayerWeightResolver.java:20-110 names, the Metal bridge's
 * upload-once registration (GgufMetalBridge.java:701-749). Files with
 * per-head norms, post norms, RoPE frequency tensors, partial RoPE or biases
 * give -3: the step does not apply them. */
int aljabr_rocm_llama_create_gguf(const char *path, int max_batch, int max_seq, aljabr_rocm_llama **out);
/* A session from a safetensors file with Hugging Face Llama names
 * (model.embed_tokens, model.layers.N.{input_layernorm, self_attn.{q,k,v,o}_proj,
 * post_attention_layernorm, mlp.{gate,up,down}_proj}, model.norm, lm_head,
 * absent: tied), architecture from `cfg` (nf4_block is forced to 128).
 * Projections and the LM head are NF4 pairs "<name>.qweight" U8 +
 * "<name>.scales" F32 (AccelWeightBridge.java:184-222) or dense ".weight"
 * F32/F16/BF16 (BF16 widened to fp32); norms and the embedding dense. Q/K
 * rows are used as stored (the step's RoPE rotates (i, i + head_dim/2)).
 * Per-head norms or biases give -3. Weights are uploaded once into memory the
 * session owns. */
int aljabr_rocm_llama_create_safetensors(const char *path, const aljabr_rocm_llama_config *cfg,
                                         aljabr_rocm_llama **out);
/* The session's configuration (e.g. of a session made from a file). */
int aljabr_rocm_llama_config_get(const aljabr_rocm_llama *m, aljabr_rocm_llama_config *cfg);

/* aljabr_rocm_llama_decode replayed from a HIP graph of the whole step: the
 * first call for a batch size (and logits buffer) runs the step and captures
 * it; later calls copy tokens and positions into the session, replay the
 * graph and copy the next tokens out (three submissions instead of one per
 * kernel). Same results as aljabr_rocm_llama_decode; the stream must not be
 * the null stream. No counterpart in the reference (the Metal runner issues
 * per-op dispatches, MTLC/aljabr_metal_matvec_api.h:161-217). */
int aljabr_rocm_llama_decode_graph(aljabr_rocm_llama *model, const void *tokens,
                                   const void *positions, int batch, void *logits,
                                   void *next_tokens);
/* Device time and algorithmic HBM bytes of one launch group of a decode step. */
typedef struct aljabr_rocm_kernel_stat {
    char name[48];          /* launch group, e.g. "attention" or "lm_head_f16" */
    int32_t launches;       /* launches of this group in the step */
    double us;              /* their summed device time in the step, microseconds */
    double bytes;           /* algorithmic bytes they move (weights, activations, KV rows read and written) */
} aljabr_rocm_kernel_stat;

/* aljabr_rocm_llama_decode with a HIP event after every launch group: runs one
 * step, waits for it, and fills up to `cap` stats aggregated by group name
 * (*count = groups found). The events add a few microseconds per group, so the
 * sum is above an unprofiled step. No counterpart in the reference: it is the
 * per-kernel roofline breakdown of the decode step. */
int aljabr_rocm_llama_decode_profile(aljabr_rocm_llama *model, const void *tokens,
                                     const void *positions, int batch, void *logits,
                                     void *next_tokens, aljabr_rocm_kernel_stat *stats,
                                     int cap, int *count);
/* Device pointer of the session's final hidden state [batch][dim] fp32. */
int aljabr_rocm_llama_hidden(aljabr_rocm_llama *model, void **hidden);
/* Device pointers of the fp16 K and V caches, each
 * [layers][max_batch][n_kv_heads][max_seq][head_dim], for loading a prefix
 * (the role of KVCacheSession's committed prefix, core/aljabr-core/.../cache/KVCacheSession.java:95-105). */
int aljabr_rocm_llama_kv_cache(aljabr_rocm_llama *model, void **k_cache, void **v_cache);

/* ======================================================================== */
/* Registered whole-step decode and fused layers (the Metal ABI's            */
/* MTLC/aljabr_metal_matvec_api.h:161-282, which the GGUF runner binds:      */
/* GJB/GgufMetalDecodeRegistration.java:17-146, GgufDecodePass.java:124-245) */
/* ======================================================================== */
/*
 * One process-wide model, as the reference keeps it: a KV cache, norm slots,
 * per-layer weights and the output registered once, then one call per token.
 * Calls are serialised and each is finished on the calling thread's stream
 * before it returns. Every data pointer may be host or device memory: device
 * weights and norms are used in place and must stay valid; host weights are
 * uploaded on first use and cached by address until
 * aljabr_rocm_reset_decode_state or aljabr_rocm_shutdown (do not change them
 * in place); host norms are copied when registered; inputs are copied in and
 * outputs copied back each call. Weight types: ALJABR_ROCM_TYPE_F32, F16,
 * Q4_0, Q8_0, Q4_K, Q6_K (the reference also takes BF16; -3 here). Failures
 * return the library's negative statuses (the reference's own negative codes
 * differ per function; its callers test rc == 0 or rc >= 0).
 */

/* fp32 caches of nLayers layers, [maxSeq][layerStrides[l]] each, zeroed
 * (aljabr_metal_init_kv_cache, MTLC/aljabr_metal_matvec_api.m:3282-3304).
 * Up to 256 layers (the reference: 64). */
int aljabr_rocm_init_kv_cache(int nLayers, int maxSeq, const int *layerStrides);
/* Copies seqLen rows of a layer's K and/or V prefix (either may be NULL)
 * into its cache (MTLC/aljabr_metal_matvec_api.m:3306-3316). */
int aljabr_rocm_sync_kv_cache(int layer, int seqLen, const float *kData, const float *vData);
/* Norm slot weights, every layer's row back to back: 0 post-attention, 1
 * FFN, 2 post-FFN, 3 attention norm ([layers][dim]); 4 Q and 5 K head norms
 * ([layers][max head_dim]) (MTLC/aljabr_metal_matvec_api.m:3318-3327). */
int aljabr_rocm_register_norm_buffer(int slot, const void *ptr, size_t bytes);
/* RoPE divisors of a layer: pair i's angle is divided by freqData[i] when it
 * is positive (MTLC/aljabr_metal_matvec_api.m:3329-3346). */
int aljabr_rocm_register_rope_freqs(int layer, const float *freqData, int freqLen);
/* One decoder layer (MTLC/aljabr_metal_matvec_api.m:3348-3425): wK NULL
 * shares the cache of the kvLayerIndex chain's first layer with K; wK
 * without wV uses the raw K projection as V. n0 = wO_K = nH*headDim, n1 = n2
 * = nKVH*headDim, wO_N the model width. attnScale <= 0: 1 with head norms,
 * else 1/sqrt(headDim). outScale applies when positive and not 1. The decode
 * step needs each layer's stride equal to nKVH*headDim (-3 otherwise). */
int aljabr_rocm_register_decode_layer(int layer, int kvLayerIndex, const void *wQ, const void *wK, const void *wV,
                                      const void *wO, const void *gate, const void *up, const void *down, int typeQ,
                                      int typeK, int typeV, int typeWO, int typeGate, int typeUp, int typeDown, int n0,
                                      int n1, int n2, int wO_K, int wO_N, int ffnDim, int nH, int nKVH, int headDim,
                                      int stride, float freqBase, int isSwa, float outScale, float attnScale,
                                      int hasPostAttnNorm, int hasPostFfnNorm, int hasQNorm, int hasKNorm,
                                      int hasUnitVNorm);
/* Output norm [outputK] and projection [outputN][outputK]; cap > 0 applies
 * cap * tanh(logit / cap) (MTLC/aljabr_metal_matvec_api.m:3427-3455). */
int aljabr_rocm_register_output(const float *outputNormW, const void *outputW, int typeOutputW, int outputK,
                                int outputN, float cap);
/* Token embedding [vocab = registered outputN][dim], rows multiplied by
 * scale (MTLC/aljabr_metal_matvec_api.m:4090-4118; the reference decodes
 * Q4_K only, this takes every weight type above). */
int aljabr_rocm_register_token_embd(const void *embdW, int typeEmbdW, int dim, float scale);
/* One token through every registered layer and the logits
 * (aljabr_metal_decode_step, MTLC/aljabr_metal_matvec_api.m:3574-4083,
 * :4121-4137): x_in [dim] is the layer-0 input; sliding-window layers see
 * the last slidingWindow positions (<= 0: all). Writes logits_out [outputN]
 * when not NULL and returns the greedy token (0 when no output is
 * registered) or a negative status. The FFN activation is the reference
 * step's tanh GELU unless aljabr_rocm_set_decode_activation says otherwise. */
int aljabr_rocm_decode_step(int pos, int slidingWindow, float eps, const float *x_in, float *logits_out);
/* The same from a token id through the registered embedding. */
int aljabr_rocm_decode_step_token(int pos, int slidingWindow, float eps, int tokenId, float *logits_out);
/* The FFN activation of the registered decode step and of nothing else: 2
 * tanh GELU (the reference step's, the default), 1 SiLU. No counterpart in
 * the reference, whose step always applies GELU (MTLC/aljabr_metal_matvec_api.m:
 * 3902-3953); SiLU models (Llama) need it. */
int aljabr_rocm_set_decode_activation(int activationKind);
/* Forget the registered model and free everything it holds (caches, norm
 * copies, uploads, activations). No counterpart in the reference, whose
 * registry only grows. */
int aljabr_rocm_reset_decode_state(void);
/* x[wO_N] = layer residual: xb = wO . attn_full, optional post-attention
 * norm, x += xb, FFN over ffnNorm(x) with activationKind (1 SiLU, 2 GELU),
 * optional post-FFN norm, x += xb, x *= outScale; then, with hasNext and
 * nextWQ, the next layer's attention norm and Q/K/V into nextQ/nextK/nextV
 * (aljabr_metal_wo_ffn_next_qkv_fused, MTLC/aljabr_metal_matvec_api.m:
 * 2198-2658). */
int aljabr_rocm_wo_ffn_next_qkv_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K,
                                      int wO_N, const float *postAttnW, int hasPostAttnNorm, const float *ffnNormW,
                                      const float *postFfnW, int hasPostFfnNorm, float eps, float outScale,
                                      const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                                      int typeDown, int ffnDim, int activationKind, int hasNext,
                                      const float *nextAttnNormW, float *nextQ, float *nextK, float *nextV,
                                      const void *nextWQ, const void *nextWK, const void *nextWV, int nextTypeQ,
                                      int nextTypeK, int nextTypeV, int nextN0, int nextN1, int nextN2);
/* The layer alone, outScale 1; the addOne flags are ignored as the
 * reference ignores them (MTLC/aljabr_metal_matvec_api.m:2660-2675). */
int aljabr_rocm_wo_ffn_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K, int wO_N,
                             const float *postAttnW, int hasPostAttnNorm, int addOnePostAttn, const float *ffnNormW,
                             int addOneFfnNorm, const float *postFfnW, int hasPostFfnNorm, int addOnePostFfn, float eps,
                             const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                             int typeDown, int ffnDim, int activationKind);
/* The last layer, then the output norm, logits [outputN] and softcap cap
 * (outputK must equal wO_N); x gets the residual when not NULL
 * (MTLC/aljabr_metal_matvec_api.m:2704-3145). */
int aljabr_rocm_wo_ffn_logits_fused(float *x, const float *attn_full, const void *wO, int typeWO, int wO_K, int wO_N,
                                    const float *postAttnW, int hasPostAttnNorm, const float *ffnNormW,
                                    const float *postFfnW, int hasPostFfnNorm, float eps, float outScale,
                                    const void *gateW, const void *upW, const void *downW, int typeGate, int typeUp,
                                    int typeDown, int ffnDim, int activationKind, const float *outputNormW,
                                    const void *outputW, int typeOutputW, int outputK, int outputN, float *logits,
                                    float cap);
/* A no-op: each call owns its residual (MTLC/aljabr_metal_matvec_api.m:2677). */
void aljabr_rocm_wo_ffn_reset_x(void);
/* The registered layer's wO + norms + FFN + residual + outScale for
 * batchSize rows: x [batchSize][wO_N] in and out, attn_full
 * [batchSize][wO_K] (aljabr_metal_wo_ffn_fused_layer_batch,
 * MTLC/aljabr_metal_matvec_api.m:4202-4350). */
int aljabr_rocm_wo_ffn_fused_layer_batch(float *x, const float *attn_full, int layer, int batchSize, float eps,
                                         int activationKind);

#ifdef __cplusplus
}
#endif
#endif
