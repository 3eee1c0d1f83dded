// kernels.hpp - stream-ordered enqueue functions shared between the C-ABI
// entry points and the decode-step driver. None of them synchronises; each
// returns an ALJABR_ROCM_* status.
#pragma once

#include <cstdint>

namespace aljabr {

struct AttnParams {
    float *out;             // [B][Hq][Sq][D] fp32
    const float *q;         // [B][Hq][Sq][D] fp32
    const void *k, *v;      // [B][Hkv][cap][D], fp16 or fp32
    const float *mask;      // [Sq][Sk] additive, or null
    const int *kv_len;      // per-batch visible key count (device), or null for Sk
    int B, Hq, Hkv, Sq, Sk, D, cap;
    float scale;
    int causal;
    int kv_f16;
};

int enqueue_attention(const AttnParams &p);

// C[M][N] = A[M][K] . W[N][K]^T for any M (slices or MFMA chosen inside).
int enqueue_matmul_nf4(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs, int M);
int enqueue_matmul_gguf(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M);
// K-split tile kernels for M <= 2 (ALJABR_ROCM_ERR_UNSUPPORTED when the shape
// or alignment does not fit them; nothing is enqueued then).
int enqueue_nf4_tile(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M);
int enqueue_gguf_tile(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M);
// Batch-1 NF4 kernel: T rows per workgroup, one wave per 2048-element K
// chunk (K <= 16384, K % 2048 == 0, block size >= 32).
int enqueue_nf4_rows(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift);
// Batch-1 NF4/Q4_0/Q8_0 kernel with a 256-entry pair table for 4-bit codes
// (K % 2048 == 0, K <= 16384; NF4 block size >= 32, 16-byte aligned codes;
// GGUF rows 4-byte aligned). `type` is an ALJABR_ROCM_TYPE_* id.
int enqueue_rows(float *C, const float *A, const uint8_t *W, const float *absmax, int K, int N, int type,
                 int bs_shift);
// NF4 small-M GEMM on MFMA (2 <= M <= 64, K % 512 == 0, block size 64).
int enqueue_nf4_mfma(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift,
                     int M);
// Persistent double-buffered batch-1 kernels (K <= 16384).
int enqueue_nf4_stream(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs_shift);
int enqueue_gguf_stream(float *C, const float *A, const uint8_t *B, int K, int N, int type);
// Small-M (M <= 8) wavefront-reduction kernels.
int enqueue_nf4_small(float *C, const float *A, const uint8_t *Bq, const float *absmax, int K, int N, int bs, int M);
int enqueue_gguf_small(float *C, const float *A, const uint8_t *B, int K, int N, int type, int M);

int enqueue_rmsnorm(float *out, const float *x, const float *w, int rows, int len, float eps);
int enqueue_rope(float *x, const int *pos, int rows, int n_heads, int head_dim, float base);
int enqueue_swiglu(float *dst, const float *gate, const float *up, long long n);
int enqueue_add(float *a, const float *b, long long n);
int enqueue_argmax(int *out, const float *x, int rows, int cols);
int enqueue_embed(float *x, const float *embed, const int *tokens, int batch, int dim, int vocab);
int enqueue_kv_append(uint16_t *cache, const float *src, const int *pos, int batch, int n_kv, int head_dim, int cap);

}  // namespace aljabr
